// Fused-time LIF / ALIF recurrence (forward) and reverse-time surrogate
// adjoint with chunked recompute (backward) for gfx950.
//
// Layout: x, spikes, grad tensors are time-major [T, BN] fp32 (BN = B*N).
// One lane owns V adjacent neurons for all T steps; membrane (and
// adaptation) live in registers for the whole launch, so HBM sees exactly
// one read of x and one write of spikes per neuron-step in the forward.
//
// Forward: the time loop is software-pipelined -- the U inputs of the next
// block of steps are in flight while the current block is computed -- so a
// lane keeps U*V*4 bytes of loads outstanding (x does not depend on the
// state, only the arithmetic is serial in t).
//
// Backward: chunks of C steps are walked in reverse.  For each chunk the
// lane reloads its checkpointed state, recomputes the C forward steps from
// x (registers hold m' and c = slope*(m'-th) per step), then runs the
// adjoint backwards through the chunk.  The x loads of the previous chunk
// and the grad_spikes loads of the current chunk are issued before the
// dependent arithmetic so each lane has ~2*C*V loads in flight.
//
// fp32 rounding: build with -ffp-contract=off; every multiply and add is
// rounded separately in the order myelin's torch backend evaluates it
// (neurons.py:111-127, functional.py:140-187).

#include "common.h"

#ifndef MYELIN_FWD_VEC
#define MYELIN_FWD_VEC 2
#endif
#ifndef MYELIN_FWD_UNROLL
#define MYELIN_FWD_UNROLL 8
#endif
#ifndef MYELIN_BWD_VEC
#define MYELIN_BWD_VEC 2
#endif

namespace {

using myelin::kWave;

typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <int V>
__device__ __forceinline__ void ld_stream(float (&r)[V], const float *p) {
  if constexpr (V == 1) {
    r[0] = __builtin_nontemporal_load(p);
  } else if constexpr (V == 2) {
    f2 t = __builtin_nontemporal_load(reinterpret_cast<const f2 *>(p));
    r[0] = t.x;
    r[1] = t.y;
  } else {
    f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
    r[0] = t.x;
    r[1] = t.y;
    r[2] = t.z;
    r[3] = t.w;
  }
}

template <int V>
__device__ __forceinline__ void st_stream(float *p, const float (&r)[V]) {
  if constexpr (V == 1) {
    __builtin_nontemporal_store(r[0], p);
  } else if constexpr (V == 2) {
    f2 t = {r[0], r[1]};
    __builtin_nontemporal_store(t, reinterpret_cast<f2 *>(p));
  } else {
    f4 t = {r[0], r[1], r[2], r[3]};
    __builtin_nontemporal_store(t, reinterpret_cast<f4 *>(p));
  }
}

template <int V>
__device__ __forceinline__ void ld(float (&r)[V], const float *p) {
  if constexpr (V == 1) {
    r[0] = *p;
  } else if constexpr (V == 2) {
    f2 t = *reinterpret_cast<const f2 *>(p);
    r[0] = t.x;
    r[1] = t.y;
  } else {
    f4 t = *reinterpret_cast<const f4 *>(p);
    r[0] = t.x;
    r[1] = t.y;
    r[2] = t.z;
    r[3] = t.w;
  }
}

template <int V>
__device__ __forceinline__ void st(float *p, const float (&r)[V]) {
  if constexpr (V == 1) {
    *p = r[0];
  } else if constexpr (V == 2) {
    f2 t = {r[0], r[1]};
    *reinterpret_cast<f2 *>(p) = t;
  } else {
    f4 t = {r[0], r[1], r[2], r[3]};
    *reinterpret_cast<f4 *>(p) = t;
  }
}

struct FwdArgs {
  const float *x;
  const float *m0;
  const float *a0;
  float *m_final;
  float *a_final;
  float *spikes;
  int32_t *packed;
  float *ckpt_m;
  float *ckpt_a;
  int64_t T, B, N, BN, W;
  float decay, rho, thr, beta, reset, slope;
  int64_t chunk;
};

// ---------------------------------------------------------------------------
// The surrogate primitives and their autograd backward, op by op.
//
// sg_smooth<SID>(c) is sigma(c) of surrogates.py:29-75 with every operation
// rounded to fp32 in the order torch evaluates the expression (scalars are
// fp32; `x / scalar` is a true division, as ATen's CPU kernel does it).
// sg_grad_autograd<SID>(c, g) is dL/dc for dL/dsigma = g, evaluated as
// torch autograd differentiates that expression: the derivative formula of
// each primitive op, applied from the output back, and a tensor used twice
// summing its two gradients.  The operations are IEEE-exact for
// fast_sigmoid, superspike and triangular.  sigmoid, atan and
// multi_gaussian also need exp / atan / erf: these are evaluated in double
// and rounded once (the fp32 value nearest the true one), which is what
// the host's vectorised fp32 versions return for all but a small fraction
// of arguments (about 1 % for exp, 2 % for erf, 1e-4 for atan); where they
// differ, the last bit differs.
// ---------------------------------------------------------------------------
constexpr float kPiF = 3.14159265358979323846f;

__device__ __forceinline__ float exp_rn(float x) { return static_cast<float>(exp(static_cast<double>(x))); }
__device__ __forceinline__ float atan_rn(float x) { return static_cast<float>(atan(static_cast<double>(x))); }
__device__ __forceinline__ float erf_rn(float x) { return static_cast<float>(erf(static_cast<double>(x))); }

__device__ __forceinline__ float sign_of(float c) { return c > 0.0f ? 1.0f : (c < 0.0f ? -1.0f : 0.0f); }

// 0.5 * (1 + erf((c - mean) / (sqrt(2) * sigma)))  (surrogates.py:61-62)
__device__ __forceinline__ float normal_cdf(float c, float mean, float k) {
  const float z = (c - mean) / k;
  return 0.5f * (1.0f + erf_rn(z));
}

template <int SID>
__device__ __forceinline__ float sg_smooth(float c) {
  if constexpr (SID == MYELIN_SG_SIGMOID) {
    return 1.0f / (1.0f + exp_rn(-c));
  } else if constexpr (SID == MYELIN_SG_FAST_SIGMOID) {
    // 0.5 * (c / (1 + |c|) + 1)
    const float b = 1.0f + fabsf(c);
    const float q = myelin::div_by(c, b, myelin::recip_rn(b));
    return 0.5f * (q + 1.0f);
  } else if constexpr (SID == MYELIN_SG_ATAN) {
    // atan(pi * c / 2) / pi + 0.5
    const float p = (c * kPiF) / 2.0f;
    return atan_rn(p) / kPiF + 0.5f;
  } else if constexpr (SID == MYELIN_SG_TRIANGULAR) {
    // (1 - |c|).clamp(0, 1)
    return fminf(fmaxf(1.0f - fabsf(c), 0.0f), 1.0f);
  } else if constexpr (SID == MYELIN_SG_SUPERSPIKE) {
    // c / (1 + |c|) + 0.5
    const float b = 1.0f + fabsf(c);
    return myelin::div_by(c, b, myelin::recip_rn(b)) + 0.5f;
  } else {
    // 0.6 * cdf(c; 0, 0.5) + 0.2 * cdf(c; 1, 1) + 0.2 * cdf(c; -1, 1),
    // sqrt(2) * sigma formed in double, as Python does, then rounded
    const float center = 0.6f * normal_cdf(c, 0.0f, static_cast<float>(1.4142135623730951 * 0.5));
    const float right = 0.2f * normal_cdf(c, 1.0f, static_cast<float>(1.4142135623730951));
    const float left = 0.2f * normal_cdf(c, -1.0f, static_cast<float>(1.4142135623730951));
    return (center + right) + left;
  }
}

// d/dc of erf's argument chain: 2/sqrt(pi) * exp(-z^2) * g, then / k
// (the erf and true-division backward formulas)
__device__ __forceinline__ float normal_cdf_grad(float c, float mean, float k, float w, float g) {
  const float z = (c - mean) / k;
  const float gh = g * w;     // w * cdf(...)
  const float gn = gh * 0.5f;  // 0.5 * (1 + erf(z))
  const float ez = exp_rn(-(z * z));
  const float gz = (static_cast<float>(1.1283791670955126) * ez) * gn;
  return gz / k;
}

template <int SID>
__device__ __forceinline__ float sg_grad_autograd(float c, float g) {
  if constexpr (SID == MYELIN_SG_SIGMOID) {
    // sigmoid_backward: g * (1 - y) * y
    const float y = sg_smooth<SID>(c);
    return (g * (1.0f - y)) * y;
  } else if constexpr (SID == MYELIN_SG_FAST_SIGMOID || SID == MYELIN_SG_SUPERSPIKE) {
    // q = c / b, b = 1 + |c|: dq/dc = 1/b (numerator) and
    // -q/b * sign(c) (denominator through abs), summed.  q/b has the sign
    // of c (and is 0 where c is), so ((-gq) * (q/b)) * sign(c) is
    // (-gq) * |q/b| exactly: a sign flip commutes with rounding.
    const float b = 1.0f + fabsf(c);
    const float y = myelin::recip_rn(b);
    const float gq = (SID == MYELIN_SG_FAST_SIGMOID) ? g * 0.5f : g;
    const float q = myelin::div_by(c, b, y);
    return myelin::div_by(gq, b, y) + (-gq) * fabsf(myelin::div_by(q, b, y));
  } else if constexpr (SID == MYELIN_SG_ATAN) {
    // (/ pi) -> atan: g / (p^2 + 1) -> (/ 2) -> (* pi)
    const float p = (c * kPiF) / 2.0f;
    const float g_at = g / kPiF;
    const float g_p = g_at / (p * p + 1.0f);
    return (g_p / 2.0f) * kPiF;
  } else if constexpr (SID == MYELIN_SG_TRIANGULAR) {
    // clamp passes g where min <= r <= max; rsub negates; abs: * sign(c)
    const float r = 1.0f - fabsf(c);
    const float g_r = (r >= 0.0f && r <= 1.0f) ? g : 0.0f;
    return (-g_r) * sign_of(c);
  } else {
    const float g_center = normal_cdf_grad(c, 0.0f, static_cast<float>(1.4142135623730951 * 0.5), 0.6f, g);
    const float g_right = normal_cdf_grad(c, 1.0f, static_cast<float>(1.4142135623730951), 0.2f, g);
    const float g_left = normal_cdf_grad(c, -1.0f, static_cast<float>(1.4142135623730951), 0.2f, g);
    // autograd reaches c through the last-built branch first
    return (g_right + g_left) + g_center;
  }
}

constexpr bool rule_autograd(int rule) { return rule >= MYELIN_RULE_STRAIGHT_THROUGH; }

// Spike value of the straight-through (hard_surrogate_spike) or smooth rule
// from the primitive's value sm = sigma(c).
template <int RULE>
__device__ __forceinline__ float spike_value(float c, float sm) {
  if constexpr (RULE >= MYELIN_RULE_SMOOTH) {
    return sm;
  } else {
    const float h = c >= 0.0f ? 1.0f : 0.0f;
    return (h + sm) - sm;
  }
}

template <int RULE>
__device__ __forceinline__ float autograd_spike(float c) {
  return spike_value<RULE>(c, sg_smooth<RULE & 15>(c));
}

// fast_sigmoid and superspike divide three numerators by b = 1 + |c| per
// step (c in the primitive, q and the upstream gradient in its backward):
// the backward shares one reciprocal myelin::recip_rn(b) between them
// (myelin::div_by, the IEEE quotient for numerators of magnitude >= 2^-100;
// a smaller one only ever meets a term it cannot change).
constexpr bool sg_quotient_form(int sid) {
  return sid == MYELIN_SG_FAST_SIGMOID || sid == MYELIN_SG_SUPERSPIKE;
}


// sigma(c) from q = c / (1 + |c|)
template <int SID>
__device__ __forceinline__ float sg_from_quotient(float q) {
  if constexpr (SID == MYELIN_SG_FAST_SIGMOID) {
    return 0.5f * (q + 1.0f);
  } else {
    return q + 0.5f;
  }
}

// One neuron step.  Returns the spike value; updates m (and a for ALIF).
template <bool ALIF, int RULE>
__device__ __forceinline__ float neuron_step(float &m, float &a, float x, const FwdArgs &p) {
  float mp = m * p.decay;
  mp = mp + x;
  float th = p.thr;
  if constexpr (ALIF) {
    float ba = p.beta * a;
    th = p.thr + ba;
  }
  float s;
  if constexpr (rule_autograd(RULE)) {
    // m'*(1 - s) + reset*s ; a*rho + s
    const float c = p.slope * (mp - th);
    s = autograd_spike<RULE>(c);
    const float keep = mp * (1.0f - s);
    m = keep + p.reset * s;
  } else {
    bool h;
    if constexpr (RULE == MYELIN_RULE_THRESHOLD) {
      h = mp >= th;
    } else {
      float c = p.slope * (mp - th);
      h = c >= 0.0f;
    }
    m = h ? p.reset : mp;
    s = h ? 1.0f : 0.0f;
  }
  if constexpr (ALIF) {
    float ra = a * p.rho;
    a = ra + s;
  }
  return s;
}

// Generic dense forward: any chunk length, every step guarded.
template <bool ALIF, int RULE, int V, int U>
__global__ __launch_bounds__(256) void fwd_dense_generic(FwdArgs p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t base = gid * V;
  if (base >= p.BN) return;
  const int64_t T = p.T, BN = p.BN;

  float m[V], a[V];
  ld<V>(m, p.m0 + base);
  if constexpr (ALIF) {
    ld<V>(a, p.a0 + base);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) a[v] = 0.0f;
  }

  float nxt[U][V];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (u < T) ld_stream<V>(nxt[u], p.x + u * BN + base);

  int64_t cc = 0;  // position inside the current checkpoint chunk
  for (int64_t t0 = 0; t0 < T; t0 += U) {
    float cur[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < V; ++v) cur[u][v] = nxt[u][v];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + U + u;
      if (t < T) ld_stream<V>(nxt[u], p.x + t * BN + base);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + u;
      if (t < T) {
        if (p.ckpt_m != nullptr && cc == 0) {
          const int64_t k = t / p.chunk;
          st<V>(p.ckpt_m + k * BN + base, m);
          if constexpr (ALIF) st<V>(p.ckpt_a + k * BN + base, a);
        }
        cc = (cc + 1 == p.chunk) ? 0 : cc + 1;
        float sp[V];
#pragma unroll
        for (int v = 0; v < V; ++v) sp[v] = neuron_step<ALIF, RULE>(m[v], a[v], cur[u][v], p);
        st_stream<V>(p.spikes + t * BN + base, sp);
      }
    }
  }
  st<V>(p.m_final + base, m);
  if constexpr (ALIF) st<V>(p.a_final + base, a);
}

// U steps starting at t0, all inside [0, T): straight-line code.
template <bool ALIF, int RULE, int V, int U>
__device__ __forceinline__ void fwd_block(const FwdArgs &p, int64_t base, int64_t t0, const float (&cur)[U][V],
                                          float (&m)[V], float (&a)[V]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float sp[V];
#pragma unroll
    for (int v = 0; v < V; ++v) sp[v] = neuron_step<ALIF, RULE>(m[v], a[v], cur[u][v], p);
    st_stream<V>(p.spikes + (t0 + u) * p.BN + base, sp);
  }
}

template <bool ALIF, int V>
__device__ __forceinline__ void fwd_ckpt(const FwdArgs &p, int64_t base, int64_t k, const float (&m)[V],
                                         const float (&a)[V]) {
  st<V>(p.ckpt_m + k * p.BN + base, m);
  if constexpr (ALIF) st<V>(p.ckpt_a + k * p.BN + base, a);
}

// The last T % U steps (rem, uniform) from registers loaded ahead: step
// t0 + u for u < rem, checkpoints as in the loop.
template <bool ALIF, int RULE, int V, int U>
__device__ __forceinline__ void fwd_tail(const FwdArgs &p, int64_t base, int64_t t0, int rem,
                                         const float (&cur)[U][V], float (&m)[V], float (&a)[V], int64_t &next_ck,
                                         int64_t &k) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u < rem) {  // uniform
      const int64_t t = t0 + u;
      if (p.ckpt_m != nullptr && t == next_ck) {
        fwd_ckpt<ALIF, V>(p, base, k++, m, a);
        next_ck += p.chunk;
      }
      float sp[V];
#pragma unroll
      for (int v = 0; v < V; ++v) sp[v] = neuron_step<ALIF, RULE>(m[v], a[v], cur[u][v], p);
      st_stream<V>(p.spikes + t * p.BN + base, sp);
    }
  }
}

// Dense-spike forward, lane owns neurons [V*gid, V*gid + V) of the flat BN
// axis.  Checkpoints (when requested) fall on block starts (chunk % U == 0,
// checked by the host), so every full block of U steps is straight-line code:
// the compiler keeps the next block's U loads in flight across the current
// block with exact vmcnt waits.  The last T % U steps are loaded in one batch
// before the last full block runs, so they wait for one load latency rather
// than one per step.
template <bool ALIF, int RULE, int V, int U>
__global__ __launch_bounds__(256) void fwd_dense(FwdArgs p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t base = gid * V;
  if (base >= p.BN) return;
  const int64_t T = p.T, BN = p.BN;
  const bool ck = p.ckpt_m != nullptr;

  float m[V], a[V];
  ld<V>(m, p.m0 + base);
  if constexpr (ALIF) {
    ld<V>(a, p.a0 + base);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) a[v] = 0.0f;
  }

  const int64_t Tm = (T / U) * U;
  const int rem = static_cast<int>(T - Tm);
  int64_t next_ck = 0, k = 0;  // next checkpoint step and its row
  float tl[U][V];              // the tail's steps
  auto load_tail = [&]() {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (u < rem) ld_stream<V>(tl[u], p.x + (Tm + u) * BN + base);  // uniform
  };
  if (Tm > 0) {
    float nxt[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) ld_stream<V>(nxt[u], p.x + u * BN + base);
    int64_t t0 = 0;
    for (; t0 + U < Tm; t0 += U) {
      float cur[U][V];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < V; ++v) cur[u][v] = nxt[u][v];
#pragma unroll
      for (int u = 0; u < U; ++u) ld_stream<V>(nxt[u], p.x + (t0 + U + u) * BN + base);
      if (ck && t0 == next_ck) {
        fwd_ckpt<ALIF, V>(p, base, k++, m, a);
        next_ck += p.chunk;
      }
      fwd_block<ALIF, RULE, V, U>(p, base, t0, cur, m, a);
    }
    load_tail();
    if (ck && t0 == next_ck) {
      fwd_ckpt<ALIF, V>(p, base, k++, m, a);
      next_ck += p.chunk;
    }
    fwd_block<ALIF, RULE, V, U>(p, base, t0, nxt, m, a);
  } else {
    load_tail();
  }
  fwd_tail<ALIF, RULE, V, U>(p, base, Tm, rem, tl, m, a, next_ck, k);
  st<V>(p.m_final + base, m);
  if constexpr (ALIF) st<V>(p.a_final + base, a);
}

// Packed-spike forward: lanes map to (b, word, bit) so that each half-wave
// owns one output word; a wave ballot yields two words per step.  Neurons
// past N in the last word of a row are inactive (their bits are 0).
template <bool ALIF, int RULE, int U>
__global__ __launch_bounds__(256) void fwd_packed(FwdArgs p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t g = gid >> 5;  // global word index over [B, W]
  const int bit = static_cast<int>(gid & 31);
  const int64_t b = g / p.W;
  const int64_t n = (g - b * p.W) * 32 + bit;
  const bool active = (b < p.B) && (n < p.N);
  const int64_t flat = b * p.N + n;
  const int64_t T = p.T, BN = p.BN;
  const int64_t words_per_step = p.B * p.W;
  // rows of an even word count from an 8-byte aligned base: the wave's two
  // words (g_wave is even) are one aligned 8-byte store
  const bool pair = words_per_step % 2 == 0 && (reinterpret_cast<uintptr_t>(p.packed) & 7) == 0;
  const int lane = static_cast<int>(threadIdx.x & (kWave - 1));
  // the wave's first word; waves start at multiples of 64 lanes, i.e. even
  // words (wave-uniform: made a scalar)
  const int64_t g_v = (gid - lane) >> 5;
  const int64_t g_wave = static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(g_v)))) |
                         (static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(g_v >> 32))) << 32);

  float m = active ? p.m0[flat] : 0.0f;
  float a = (ALIF && active) ? p.a0[flat] : 0.0f;

  float nxt[U];
#pragma unroll
  for (int u = 0; u < U; ++u) nxt[u] = (active && u < T) ? __builtin_nontemporal_load(p.x + u * BN + flat) : 0.0f;

  int64_t cc = 0;
  for (int64_t t0 = 0; t0 < T; t0 += U) {
    float cur[U];
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + U + u;
      if (t < T && active) nxt[u] = __builtin_nontemporal_load(p.x + t * BN + flat);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + u;
      if (t < T) {
        if (p.ckpt_m != nullptr && cc == 0 && active) {
          const int64_t k = t / p.chunk;
          p.ckpt_m[k * BN + flat] = m;
          if constexpr (ALIF) p.ckpt_a[k * BN + flat] = a;
        }
        cc = (cc + 1 == p.chunk) ? 0 : cc + 1;
        bool s = false;
        if (active) s = neuron_step<ALIF, RULE>(m, a, cur[u], p) != 0.0f;
        const uint64_t bits = __ballot(s);
        int32_t *row = p.packed + t * words_per_step;
        if (pair) {
          // the wave's two words as one 8-byte store, the same value from
          // every lane: no lane-selected branch a step
          if (g_wave < words_per_step) *reinterpret_cast<uint64_t *>(row + g_wave) = bits;
        } else {
          if (lane == 0 && g_wave < words_per_step) row[g_wave] = static_cast<int32_t>(bits & 0xffffffffu);
          if (lane == 32 && g_wave + 1 < words_per_step) row[g_wave + 1] = static_cast<int32_t>(bits >> 32);
        }
      }
    }
  }
  if (active) {
    p.m_final[flat] = m;
    if constexpr (ALIF) p.a_final[flat] = a;
  }
}

// ---------------------------------------------------------------------------
// surrogate derivatives sigma'(c) (surrogates.py:78-102), ids as
// triton/lif.py:356-370.
// ---------------------------------------------------------------------------
template <int SID>
__device__ __forceinline__ float sg_deriv(float c) {
  if constexpr (SID == MYELIN_SG_SIGMOID) {
    // v(1-v) written as e/(1+e)^2 with e = exp(-|c|): no cancellation
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
  } else if constexpr (SID == MYELIN_SG_NONE) {
    return 0.0f;
  } else {
    float z = c / 0.5f, r = c - 1.0f, l = c + 1.0f;
    return 0.47873073648171924f * expf(-0.5f * z * z) + 0.07978845608028655f * expf(-0.5f * r * r) +
           0.07978845608028655f * expf(-0.5f * l * l);
  }
}

struct BwdArgs {
  const float *x;
  const float *ckpt_m;
  const float *ckpt_a;
  const float *gs;
  const float *gmT;
  const float *gaT;
  float *gx;
  float *gm0;
  float *ga0;
  int64_t T, BN;
  float decay, rho, thr, beta, reset, slope;
};

// Recompute one chunk forward from its checkpointed state: pre[j] = m'_t,
// cv[j] = c_t = slope*(m'_t - th_t) (for SG_NONE: m'_t - th_t, so that
// c >= 0 is the plain threshold test).  GUARD: only the first `len` steps.
// FR: 0 for exact 0/1 spikes, else the forward's autograd rule
// (straight-through / smooth), whose spike values the reset and the
// adaptation carry.
template <bool ALIF, int C, int SID, int V, bool GUARD, int FR, bool RZ>
__device__ __forceinline__ void bwd_recompute(const BwdArgs &p, int len, const float (&xb)[C][V], float (&m)[V],
                                              float (&a)[V], float (&pre)[C][V], float (&cv)[C][V]) {
#pragma unroll
  for (int j = 0; j < C; ++j) {
    if (GUARD && j >= len) break;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float mp = m[v] * p.decay;
      mp = mp + xb[j][v];
      float th = p.thr;
      if constexpr (ALIF) {
        float ba = p.beta * a[v];
        th = p.thr + ba;
      }
      const float c = (SID == MYELIN_SG_NONE) ? mp - th : p.slope * (mp - th);
      pre[j][v] = mp;
      cv[j][v] = c;
      float s;
      if constexpr (FR != 0) {
        if constexpr (sg_quotient_form(SID)) {
          // the reciprocal the reverse walk shares between its quotients
          const float b = 1.0f + fabsf(c);
          const float y = myelin::recip_rn(b);
          s = spike_value<FR>(c, sg_from_quotient<SID>(myelin::div_by(c, b, y)));
        } else {
          s = autograd_spike<FR>(c);
        }
        const float keep = mp * (1.0f - s);
        // RZ: reset == 0, whose term only adds a zero
        m[v] = RZ ? keep : keep + p.reset * s;
      } else {
        const bool h = c >= 0.0f;
        s = h ? 1.0f : 0.0f;
        m[v] = h ? p.reset : mp;
      }
      if constexpr (ALIF) {
        float ra = a[v] * p.rho;
        a[v] = ra + s;
      }
    }
  }
}

// Walk one chunk backwards, storing grad_x for t0 + j.  Per step, with
// gm = dL/dm_{t+1}, ga = dL/da_{t+1}:
//   closed form (FR == 0):
//     q  = gm*(reset - m') + gs_t + ga
//     gc = q * slope * sigma'(c)
//     gp = gm*(1 - s) + gc          -> grad_x[t]
//     ga = ga*rho - beta*gc ;  gm = gp*decay
//   autograd order (FR != 0), s the forward's spike value:
//     gS = ((gs_t + ga) + gm*reset) - gm*m'     (dL/ds, in the order the
//           stack, adaptation, reset and m'*(1 - s) nodes deliver it)
//     gd = sg_grad_autograd(c, gS) * slope      (dL/d(m' - th))
//     gp = gm*(1 - s) + gd          -> grad_x[t]
//     ga = ga*rho + (-gd)*beta ;  gm = gp*decay
// (steps J1 - 1 down to J0 of the chunk; the whole chunk by default)
template <bool ALIF, int C, int SID, int V, bool GS, bool GUARD, int FR, bool RZ, int J0 = 0, int J1 = C>
__device__ __forceinline__ void bwd_reverse(const BwdArgs &p, int64_t base, int64_t t0, int len,
                                            const float (&gsb)[C][V], const float (&pre)[C][V],
                                            const float (&cv)[C][V], float (&gm)[V],
                                            float (&ga)[V]) {
#pragma unroll
  for (int j = J1 - 1; j >= J0; --j) {
    if (GUARD && j >= len) continue;
    float g[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float c = cv[j][v];
      // The quotient forms rebuild b, 1/b, q and the spike value from c
      // here (about 12 VALU per neuron-step) instead of keeping them from
      // the recompute: the empty asm hides c's origin, so the compiler
      // cannot carry those values across the phases.  Three more values
      // per step kept live took 250 VGPRs (2 waves per SIMD) against 149
      // (3 waves); [256, 128, 4096] ALIF fast_sigmoid: 280 -> 273 us.
      if constexpr (FR != 0 && sg_quotient_form(SID)) asm volatile("" : "+v"(c));
      const float s = c >= 0.0f ? 1.0f : 0.0f;
      if constexpr (SID == MYELIN_SG_NONE) {
        // where(s, reset, m') passes gradient to m' only where s == 0
        const float gp = s != 0.0f ? 0.0f : gm[v];
        g[v] = gp;
        if constexpr (ALIF) ga[v] = ga[v] * p.rho;
        gm[v] = gp * p.decay;
      } else if constexpr (FR != 0) {
        float sv, b = 0.0f, y = 0.0f, q = 0.0f;
        if constexpr (sg_quotient_form(SID)) {
          b = 1.0f + fabsf(c);
          y = myelin::recip_rn(b);
          q = myelin::div_by(c, b, y);
          sv = spike_value<FR>(c, sg_from_quotient<SID>(q));
        } else {
          sv = autograd_spike<FR>(c);
        }
        const float G = gm[v];
        float gS;
        if constexpr (GS) {
          gS = gsb[j][v];
          if constexpr (ALIF) gS = gS + ga[v];
          if constexpr (!RZ) gS = gS + G * p.reset;
        } else if constexpr (ALIF) {
          gS = RZ ? ga[v] : ga[v] + G * p.reset;
        } else {
          gS = G * p.reset;
        }
        gS = gS - G * pre[j][v];
        float gc;
        if constexpr (sg_quotient_form(SID)) {
          // as sg_grad_autograd, with the shared reciprocal
          const float gq = (SID == MYELIN_SG_FAST_SIGMOID) ? gS * 0.5f : gS;
          gc = myelin::div_by(gq, b, y) + (-gq) * fabsf(myelin::div_by(q, b, y));
        } else {
          gc = sg_grad_autograd<SID>(c, gS);
        }
        const float gd = gc * p.slope;
        const float gp = G * (1.0f - sv) + gd;
        g[v] = gp;
        if constexpr (ALIF) {
          float r = ga[v] * p.rho;
          ga[v] = r + (-gd) * p.beta;
        }
        gm[v] = gp * p.decay;
      } else {
        const float dsdm = p.slope * sg_deriv<SID>(c);
        float q = gm[v] * (p.reset - pre[j][v]);
        if constexpr (GS) q = q + gsb[j][v];
        if constexpr (ALIF) q = q + ga[v];
        const float gc = q * dsdm;
        const float gp = gm[v] * (1.0f - s) + gc;
        g[v] = gp;
        if constexpr (ALIF) {
          float r = ga[v] * p.rho;
          ga[v] = r - p.beta * gc;
        }
        gm[v] = gp * p.decay;
      }
    }
    st_stream<V>(p.gx + (t0 + j) * p.BN + base, g);
  }
}

template <bool ALIF, int V>
__device__ __forceinline__ void bwd_load_ckpt(const BwdArgs &p, int64_t k, int64_t base, float (&m)[V],
                                              float (&a)[V]) {
  ld<V>(m, p.ckpt_m + k * p.BN + base);
  if constexpr (ALIF) {
    ld<V>(a, p.ckpt_a + k * p.BN + base);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) a[v] = 0.0f;
  }
}

// Reverse-time adjoint over chunks of C steps, lane owns V neurons.
// The partial last chunk (T % C steps) is handled first with guards; the
// full chunks then run as straight-line code, software-pipelined: the
// checkpoint and x of chunk k-1 are loaded while chunk k is walked
// backwards, and grad_spikes of chunk k while chunk k is recomputed.
template <bool ALIF, int C, int SID, int V, bool GS, int FR, bool RZ = false>
__global__ __launch_bounds__(256) void bwd_chunked(BwdArgs p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t base = gid * V;
  if (base >= p.BN) return;
  const int64_t T = p.T, BN = p.BN;
  const int64_t Kf = T / C;
  const int rem = static_cast<int>(T - Kf * C);

  float gm[V], ga[V];
  if (p.gmT != nullptr) {
    ld<V>(gm, p.gmT + base);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) gm[v] = 0.0f;
  }
  if (ALIF && p.gaT != nullptr) {
    ld<V>(ga, p.gaT + base);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) ga[v] = 0.0f;
  }

  float xb[C][V], gsb[C][V], pre[C][V], cv[C][V], m[V], a[V];
  if (rem > 0) {
    const int64_t t0 = Kf * C;
    bwd_load_ckpt<ALIF, V>(p, Kf, base, m, a);
#pragma unroll
    for (int j = 0; j < C; ++j)
      if (j < rem) ld_stream<V>(xb[j], p.x + (t0 + j) * BN + base);
    if constexpr (GS) {
#pragma unroll
      for (int j = 0; j < C; ++j)
        if (j < rem) ld_stream<V>(gsb[j], p.gs + (t0 + j) * BN + base);
    }
    bwd_recompute<ALIF, C, SID, V, true, FR, RZ>(p, rem, xb, m, a, pre, cv);
    bwd_reverse<ALIF, C, SID, V, GS, true, FR, RZ>(p, base, t0, rem, gsb, pre, cv, gm, ga);
  }
  if (Kf > 0) {
    int64_t k = Kf - 1;
    bwd_load_ckpt<ALIF, V>(p, k, base, m, a);
#pragma unroll
    for (int j = 0; j < C; ++j) ld_stream<V>(xb[j], p.x + (k * C + j) * BN + base);
    for (; k > 0; --k) {
      const int64_t t0 = k * C;
      if constexpr (C == 16) {
        // Chunks of 16 hold twice the trace of chunks of 8; issuing the
        // loads a quarter at a time, as the reverse walk frees registers,
        // keeps the live set near that of chunk 8: grad_spikes(k) of the
        // upper half | recompute(k) | ckpt, x(k-1) lower half | reverse
        // steps 15..12 | grad_spikes(k) lower half | reverse 11..8 |
        // x(k-1) upper half | reverse 7..0
        if constexpr (GS) {
#pragma unroll
          for (int j = C / 2; j < C; ++j) ld_stream<V>(gsb[j], p.gs + (t0 + j) * BN + base);
        }
        __builtin_amdgcn_sched_barrier(0);
        bwd_recompute<ALIF, C, SID, V, false, FR, RZ>(p, C, xb, m, a, pre, cv);
        __builtin_amdgcn_sched_barrier(0);
        bwd_load_ckpt<ALIF, V>(p, k - 1, base, m, a);
#pragma unroll
        for (int j = 0; j < C / 2; ++j) ld_stream<V>(xb[j], p.x + (t0 - C + j) * BN + base);
        __builtin_amdgcn_sched_barrier(0);
        bwd_reverse<ALIF, C, SID, V, GS, false, FR, RZ, 3 * C / 4, C>(p, base, t0, C, gsb, pre, cv, gm, ga);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (GS) {
#pragma unroll
          for (int j = 0; j < C / 2; ++j) ld_stream<V>(gsb[j], p.gs + (t0 + j) * BN + base);
        }
        __builtin_amdgcn_sched_barrier(0);
        bwd_reverse<ALIF, C, SID, V, GS, false, FR, RZ, C / 2, 3 * C / 4>(p, base, t0, C, gsb, pre, cv, gm, ga);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = C / 2; j < C; ++j) ld_stream<V>(xb[j], p.x + (t0 - C + j) * BN + base);
        __builtin_amdgcn_sched_barrier(0);
        bwd_reverse<ALIF, C, SID, V, GS, false, FR, RZ, 0, C / 2>(p, base, t0, C, gsb, pre, cv, gm, ga);
        __builtin_amdgcn_sched_barrier(0);
      } else {
        if constexpr (GS) {
#pragma unroll
          for (int j = 0; j < C; ++j) ld_stream<V>(gsb[j], p.gs + (t0 + j) * BN + base);
        }
        // keep the issue order: grad_spikes(k) | recompute(k) | ckpt, x(k-1) |
        // reverse(k), so the reverse phase waits only for grad_spikes(k) while
        // the loads of chunk k-1 stay in flight
        __builtin_amdgcn_sched_barrier(0);
        bwd_recompute<ALIF, C, SID, V, false, FR, RZ>(p, C, xb, m, a, pre, cv);
        __builtin_amdgcn_sched_barrier(0);
        bwd_load_ckpt<ALIF, V>(p, k - 1, base, m, a);
#pragma unroll
        for (int j = 0; j < C; ++j) ld_stream<V>(xb[j], p.x + (t0 - C + j) * BN + base);
        __builtin_amdgcn_sched_barrier(0);
        bwd_reverse<ALIF, C, SID, V, GS, false, FR, RZ>(p, base, t0, C, gsb, pre, cv, gm, ga);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (GS) {
#pragma unroll
      for (int j = 0; j < C; ++j) ld_stream<V>(gsb[j], p.gs + j * BN + base);
    }
    bwd_recompute<ALIF, C, SID, V, false, FR, RZ>(p, C, xb, m, a, pre, cv);
    bwd_reverse<ALIF, C, SID, V, GS, false, FR, RZ>(p, base, 0, C, gsb, pre, cv, gm, ga);
  }
  st<V>(p.gm0 + base, gm);
  if constexpr (ALIF) st<V>(p.ga0 + base, ga);
}

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------

int64_t blocks_for(int64_t lanes) { return (lanes + 255) / 256; }

template <bool ALIF, int RULE>
int launch_fwd(const FwdArgs &a, hipStream_t stream) {
  constexpr bool AG = rule_autograd(RULE);
  if (a.packed != nullptr) {
    if constexpr (AG) {
      return myelin::invalid("spike rule %d emits spike values; packed output takes the threshold rules", RULE);
    } else {
      const int64_t lanes = a.B * a.W * 32;
      fwd_packed<ALIF, RULE, MYELIN_FWD_UNROLL><<<dim3(blocks_for(lanes)), dim3(256), 0, stream>>>(a);
      return myelin::launched("fwd_packed");
    }
  }
  // widest vector the pointers and BN allow (at most 2 neurons per lane for
  // the autograd rules, which are built at 1 and 2)
  const void *ptrs[] = {a.x, a.m0, a.m_final, a.spikes, a.ckpt_m, ALIF ? a.a0 : nullptr,
                        ALIF ? a.a_final : nullptr, ALIF ? a.ckpt_a : nullptr};
  int v = (AG && MYELIN_FWD_VEC > 2) ? 2 : MYELIN_FWD_VEC;
  while (v > 1) {
    bool ok = (a.BN % v) == 0;
    for (const void *q : ptrs)
      if (q != nullptr && !myelin::aligned(q, 4 * v)) ok = false;
    if (ok) break;
    v >>= 1;
  }
  // Small grids (under two waves per SIMD at this width) without
  // checkpoints: one neuron per lane and 32 steps in flight, so a latency-
  // bound walk over T has twice the lanes and four times the loads outstanding.
  if (a.ckpt_m == nullptr && (a.BN + v - 1) / v < 2 * 1024 * 64) {
    fwd_dense<ALIF, RULE, 1, 4 * MYELIN_FWD_UNROLL><<<dim3(blocks_for(a.BN)), dim3(256), 0, stream>>>(a);
    return myelin::launched("fwd_dense");
  }
  const int64_t lanes = (a.BN + v - 1) / v;
  const dim3 grid(blocks_for(lanes));
  constexpr int U = MYELIN_FWD_UNROLL;
  if (a.ckpt_m != nullptr && a.chunk % U != 0) {
    if constexpr (AG) {
      fwd_dense_generic<ALIF, RULE, 1, U><<<dim3(blocks_for(a.BN)), dim3(256), 0, stream>>>(a);
    } else {
      if (v == 4)
        fwd_dense_generic<ALIF, RULE, 4, U><<<grid, dim3(256), 0, stream>>>(a);
      else if (v == 2)
        fwd_dense_generic<ALIF, RULE, 2, U><<<grid, dim3(256), 0, stream>>>(a);
      else
        fwd_dense_generic<ALIF, RULE, 1, U><<<grid, dim3(256), 0, stream>>>(a);
    }
    return myelin::launched("fwd_dense_generic");
  }
  if (v == 2)
    fwd_dense<ALIF, RULE, 2, U><<<grid, dim3(256), 0, stream>>>(a);
  else if (v == 1)
    fwd_dense<ALIF, RULE, 1, U><<<grid, dim3(256), 0, stream>>>(a);
  else if constexpr (!AG)
    fwd_dense<ALIF, RULE, 4, U><<<grid, dim3(256), 0, stream>>>(a);
  return myelin::launched("fwd_dense");
}

template <bool ALIF, int BASE>
int launch_fwd_autograd(const FwdArgs &a, int sid, hipStream_t stream) {
  switch (sid) {
    case MYELIN_SG_SIGMOID: return launch_fwd<ALIF, BASE + MYELIN_SG_SIGMOID>(a, stream);
    case MYELIN_SG_FAST_SIGMOID: return launch_fwd<ALIF, BASE + MYELIN_SG_FAST_SIGMOID>(a, stream);
    case MYELIN_SG_ATAN: return launch_fwd<ALIF, BASE + MYELIN_SG_ATAN>(a, stream);
    case MYELIN_SG_TRIANGULAR: return launch_fwd<ALIF, BASE + MYELIN_SG_TRIANGULAR>(a, stream);
    case MYELIN_SG_SUPERSPIKE: return launch_fwd<ALIF, BASE + MYELIN_SG_SUPERSPIKE>(a, stream);
    case MYELIN_SG_MULTI_GAUSSIAN: return launch_fwd<ALIF, BASE + MYELIN_SG_MULTI_GAUSSIAN>(a, stream);
    default: return myelin::invalid("unknown spike rule %d", BASE + sid);
  }
}

template <bool ALIF>
int fwd_entry(FwdArgs &a, int rule, hipStream_t stream) {
  if (a.T < 1 || a.B < 1 || a.N < 1) return myelin::invalid("T, B and N must be positive");
  if (a.x == nullptr || a.m0 == nullptr || a.m_final == nullptr)
    return myelin::invalid("x, m0 and m_final are required");
  if (ALIF && (a.a0 == nullptr || a.a_final == nullptr))
    return myelin::invalid("a0 and a_final are required for ALIF");
  if ((a.spikes == nullptr) == (a.packed == nullptr))
    return myelin::invalid("exactly one of spikes / packed must be given");
  if (a.ckpt_m != nullptr && a.chunk < 1) return myelin::invalid("chunk must be positive");
  if (ALIF && (a.ckpt_m == nullptr) != (a.ckpt_a == nullptr))
    return myelin::invalid("ckpt_m and ckpt_a must be given together");
  if (a.chunk < 1) a.chunk = 1;
  a.BN = a.B * a.N;
  a.W = (a.N + 31) / 32;
  if (rule == MYELIN_RULE_THRESHOLD) return launch_fwd<ALIF, MYELIN_RULE_THRESHOLD>(a, stream);
  if (rule == MYELIN_RULE_SURROGATE) return launch_fwd<ALIF, MYELIN_RULE_SURROGATE>(a, stream);
  if (rule >= MYELIN_RULE_SMOOTH)
    return launch_fwd_autograd<ALIF, MYELIN_RULE_SMOOTH>(a, rule - MYELIN_RULE_SMOOTH, stream);
  if (rule >= MYELIN_RULE_STRAIGHT_THROUGH)
    return launch_fwd_autograd<ALIF, MYELIN_RULE_STRAIGHT_THROUGH>(a, rule - MYELIN_RULE_STRAIGHT_THROUGH, stream);
  return myelin::invalid("unknown spike rule %d", rule);
}

// FR: 0 for the closed form, else the forward's autograd rule (the
// smooth rule's kernels are built at one neuron per lane only)
template <bool ALIF, int C, int SID, int FR>
int launch_bwd_sid(const BwdArgs &a, hipStream_t stream) {
  const void *ptrs[] = {a.x, a.ckpt_m, a.gs, a.gmT, a.gx, a.gm0, a.ckpt_a, a.gaT, a.ga0};
  int v = FR >= MYELIN_RULE_SMOOTH ? 1 : MYELIN_BWD_VEC;
  while (v > 1) {
    bool ok = (a.BN % v) == 0;
    for (const void *q : ptrs)
      if (q != nullptr && !myelin::aligned(q, 4 * v)) ok = false;
    if (ok) break;
    v >>= 1;
  }
  const bool gs = (SID != MYELIN_SG_NONE) && a.gs != nullptr;
  // without a spike gradient the two-neuron chunk-16 kernel does not fit
  // the register file (about 460 registers); one neuron per lane needs < 80.
  // The autograd-order kernels without a spike gradient are built at one
  // neuron per lane only.
  if ((C == 16 || FR != 0) && !gs) v = 1;
  const dim3 grid(blocks_for((a.BN + v - 1) / v));
  // gs implies SID != NONE, and v == 2 without gs implies C == 8 and the
  // closed form: the constexpr guards keep the unreachable instances out
  // of the library
  if (v == 2) {
    if (gs) {
      // reset == 0 (either sign): the autograd order's reset terms only add
      // zeros, so the hard-forward kernel is also built without them
      if constexpr (SID != MYELIN_SG_NONE && FR != 0 && FR < MYELIN_RULE_SMOOTH) {
        if (a.reset == 0.0f) {
          bwd_chunked<ALIF, C, SID, 2, true, FR, true><<<grid, dim3(256), 0, stream>>>(a);
          return myelin::launched("bwd_chunked");
        }
      }
      if constexpr (SID != MYELIN_SG_NONE && FR < MYELIN_RULE_SMOOTH)
        bwd_chunked<ALIF, C, SID, 2, true, FR><<<grid, dim3(256), 0, stream>>>(a);
    } else if constexpr (C != 16 && FR == 0) {
      bwd_chunked<ALIF, C, SID, 2, false, FR><<<grid, dim3(256), 0, stream>>>(a);
    }
  } else {
    if (gs) {
      if constexpr (SID != MYELIN_SG_NONE)
        bwd_chunked<ALIF, C, SID, 1, true, FR><<<grid, dim3(256), 0, stream>>>(a);
    } else {
      bwd_chunked<ALIF, C, SID, 1, false, FR><<<grid, dim3(256), 0, stream>>>(a);
    }
  }
  return myelin::launched("bwd_chunked");
}

// code: a surrogate id (closed form) or MYELIN_SG_AUTOGRAD[_SMOOTH] + id
template <bool ALIF, int C>
int launch_bwd_c(const BwdArgs &a, int code, hipStream_t stream) {
  switch (code) {
#define MYELIN_BWD_CASES(SID)                                                                          \
  case SID: return launch_bwd_sid<ALIF, C, SID, 0>(a, stream);                                       \
  case MYELIN_SG_AUTOGRAD + SID:                                                                       \
    if constexpr (C == 16)                                                                             \
      return launch_bwd_sid<ALIF, C, SID, MYELIN_RULE_STRAIGHT_THROUGH + SID>(a, stream);              \
    break;                                                                                             \
  case MYELIN_SG_AUTOGRAD_SMOOTH + SID:                                                                \
    if constexpr (C == 16) return launch_bwd_sid<ALIF, C, SID, MYELIN_RULE_SMOOTH + SID>(a, stream);   \
    break;
    MYELIN_BWD_CASES(MYELIN_SG_SIGMOID)
    MYELIN_BWD_CASES(MYELIN_SG_FAST_SIGMOID)
    MYELIN_BWD_CASES(MYELIN_SG_ATAN)
    MYELIN_BWD_CASES(MYELIN_SG_TRIANGULAR)
    MYELIN_BWD_CASES(MYELIN_SG_SUPERSPIKE)
    MYELIN_BWD_CASES(MYELIN_SG_MULTI_GAUSSIAN)
#undef MYELIN_BWD_CASES
    case MYELIN_SG_NONE: return launch_bwd_sid<ALIF, C, MYELIN_SG_NONE, 0>(a, stream);
    default: return myelin::invalid("unknown surrogate code %d", code);
  }
  return myelin::invalid("surrogate code %d (autograd order) needs chunk 16; got %d", code, C);
}

template <bool ALIF>
int bwd_entry(const BwdArgs &a, int sid, int64_t chunk, hipStream_t stream) {
  if (a.T < 1 || a.BN < 1) return myelin::invalid("T and BN must be positive");
  if (a.x == nullptr || a.ckpt_m == nullptr || a.gx == nullptr || a.gm0 == nullptr)
    return myelin::invalid("x, ckpt_m, grad_x and grad_m0 are required");
  if (ALIF && (a.ckpt_a == nullptr || a.ga0 == nullptr))
    return myelin::invalid("ckpt_a and grad_a0 are required for ALIF");
  switch (chunk) {
    case 8: return launch_bwd_c<ALIF, 8>(a, sid, stream);
    case 16: return launch_bwd_c<ALIF, 16>(a, sid, stream);
    default: return myelin::invalid("backward chunk must be 8 or 16; got %lld", (long long)chunk);
  }
}

}  // namespace

extern "C" int myelin_lif_fwd_f32(const float *x, const float *m0, float *m_final, float *spikes, int32_t *packed,
                                  float *ckpt_m, int64_t T, int64_t B, int64_t N, float decay, float threshold,
                                  float reset, float slope, int rule, int64_t chunk, myelin_stream_t stream) {
  FwdArgs a{};
  a.x = x;
  a.m0 = m0;
  a.m_final = m_final;
  a.spikes = spikes;
  a.packed = packed;
  a.ckpt_m = ckpt_m;
  a.T = T;
  a.B = B;
  a.N = N;
  a.decay = decay;
  a.thr = threshold;
  a.reset = reset;
  a.slope = slope;
  a.chunk = chunk;
  return fwd_entry<false>(a, rule, myelin::as_hip(stream));
}

extern "C" int myelin_alif_fwd_f32(const float *x, const float *m0, const float *a0, float *m_final, float *a_final,
                                   float *spikes, int32_t *packed, float *ckpt_m, float *ckpt_a, int64_t T,
                                   int64_t B, int64_t N, float decay, float rho, float threshold, float beta,
                                   float reset, float slope, int rule, int64_t chunk, myelin_stream_t stream) {
  FwdArgs a{};
  a.x = x;
  a.m0 = m0;
  a.a0 = a0;
  a.m_final = m_final;
  a.a_final = a_final;
  a.spikes = spikes;
  a.packed = packed;
  a.ckpt_m = ckpt_m;
  a.ckpt_a = ckpt_a;
  a.T = T;
  a.B = B;
  a.N = N;
  a.decay = decay;
  a.rho = rho;
  a.thr = threshold;
  a.beta = beta;
  a.reset = reset;
  a.slope = slope;
  a.chunk = chunk;
  return fwd_entry<true>(a, rule, myelin::as_hip(stream));
}

extern "C" int myelin_lif_bwd_f32(const float *x, const float *ckpt_m, const float *grad_spikes,
                                  const float *grad_m_final, float *grad_x, float *grad_m0, int64_t T, int64_t BN,
                                  float decay, float threshold, float reset, float slope, int surrogate_id,
                                  int64_t chunk, myelin_stream_t stream) {
  BwdArgs a{};
  a.x = x;
  a.ckpt_m = ckpt_m;
  a.gs = grad_spikes;
  a.gmT = grad_m_final;
  a.gx = grad_x;
  a.gm0 = grad_m0;
  a.T = T;
  a.BN = BN;
  a.decay = decay;
  a.thr = threshold;
  a.reset = reset;
  a.slope = slope;
  return bwd_entry<false>(a, surrogate_id, chunk, myelin::as_hip(stream));
}

extern "C" int myelin_alif_bwd_f32(const float *x, const float *ckpt_m, const float *ckpt_a,
                                   const float *grad_spikes, const float *grad_m_final, const float *grad_a_final,
                                   float *grad_x, float *grad_m0, float *grad_a0, int64_t T, int64_t BN, float decay,
                                   float rho, float threshold, float beta, float reset, float slope, int surrogate_id,
                                   int64_t chunk, myelin_stream_t stream) {
  BwdArgs a{};
  a.x = x;
  a.ckpt_m = ckpt_m;
  a.ckpt_a = ckpt_a;
  a.gs = grad_spikes;
  a.gmT = grad_m_final;
  a.gaT = grad_a_final;
  a.gx = grad_x;
  a.gm0 = grad_m0;
  a.ga0 = grad_a0;
  a.T = T;
  a.BN = BN;
  a.decay = decay;
  a.rho = rho;
  a.thr = threshold;
  a.beta = beta;
  a.reset = reset;
  a.slope = slope;
  return bwd_entry<true>(a, surrogate_id, chunk, myelin::as_hip(stream));
}

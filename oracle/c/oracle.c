/*
 * Plain-C restatement of myelin's fused-time neuron path.
 *
 * TEST INFRASTRUCTURE ONLY: compiled into oracle/liboracle_c.so, loaded by
 * oracle/c_ref.py from tests/, smoke() and bench.py's cpu_baseline leg.  The
 * shipped library never links it.
 *
 * Build with -ffp-contract=off: every multiply and add is rounded on its own,
 * exactly like the separate ATen ops of the reference's torch backend.
 *
 * Citations are file:line in djsaunde/myelin (src/myelin/...).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* surrogate ids follow triton/lif.py:356-370 */
enum { SG_SIGMOID = 0, SG_FAST_SIGMOID = 1, SG_ATAN = 2, SG_TRIANGULAR = 3,
       SG_SUPERSPIKE = 4, SG_MULTI_GAUSSIAN = 5 };

/* sigma'(c), surrogates.py:78-102 */
static float sg_deriv(int id, float c)
{
    switch (id) {
    case SG_SIGMOID: {
        /* v(1-v) written as e/(1+e)^2 with e = exp(-|c|): no cancellation */
        float e = expf(-fabsf(c));
        float d = 1.0f + e;
        return e / (d * d);
    }
    case SG_FAST_SIGMOID: {
        float d = 1.0f + fabsf(c);
        return 0.5f / (d * d);
    }
    case SG_ATAN: {
        float s = 1.5707963267948966f * c;
        return 0.5f / (1.0f + s * s);
    }
    case SG_TRIANGULAR: {
        float sg = (c > 0.0f) ? 1.0f : ((c < 0.0f) ? -1.0f : 0.0f);
        return fabsf(c) < 1.0f ? -sg : 0.0f;
    }
    case SG_SUPERSPIKE: {
        float d = 1.0f + fabsf(c);
        return 1.0f / (d * d);
    }
    case SG_MULTI_GAUSSIAN: {
        float z = c / 0.5f, r = c - 1.0f, l = c + 1.0f;
        return 0.47873073648171924f * expf(-0.5f * z * z)
             + 0.07978845608028655f * expf(-0.5f * r * r)
             + 0.07978845608028655f * expf(-0.5f * l * l);
    }
    default:
        return 0.0f;
    }
}

/* spike decision: plain unrolls compare m >= th (neurons.py:112,124);
 * surrogate unrolls test slope*(m - th) >= 0 (surrogates.py:108). */
static int spike_of(float m, float th, int surrogate_mode, float slope)
{
    if (surrogate_mode) {
        float c = slope * (m - th);
        return c >= 0.0f;
    }
    return m >= th;
}

/* LIF over [T, BN] (functional.py:21-45, neurons.py:106-114) */
void orc_lif_fwd(const float *x, const float *m0, float *mT, float *spikes,
                 int64_t T, int64_t BN, float decay, float thr, float reset,
                 int surrogate_mode, float slope)
{
    for (int64_t i = 0; i < BN; ++i) {
        float m = m0[i];
        for (int64_t t = 0; t < T; ++t) {
            float p = m * decay;
            m = p + x[t * BN + i];
            int s = spike_of(m, thr, surrogate_mode, slope);
            spikes[t * BN + i] = s ? 1.0f : 0.0f;
            if (s) m = reset;
        }
        mT[i] = m;
    }
}

/* ALIF (functional.py:48-78, neurons.py:117-128) */
void orc_alif_fwd(const float *x, const float *m0, const float *a0, float *mT,
                  float *aT, float *spikes, int64_t T, int64_t BN, float decay,
                  float rho, float thr, float beta, float reset,
                  int surrogate_mode, float slope)
{
    for (int64_t i = 0; i < BN; ++i) {
        float m = m0[i], a = a0[i];
        for (int64_t t = 0; t < T; ++t) {
            float p = m * decay;
            m = p + x[t * BN + i];
            float ba = beta * a;
            float th = thr + ba;
            int s = spike_of(m, th, surrogate_mode, slope);
            float sf = s ? 1.0f : 0.0f;
            spikes[t * BN + i] = sf;
            if (s) m = reset;
            float ra = a * rho;
            a = ra + sf;
        }
        mT[i] = m;
        aT[i] = a;
    }
}

/*
 * Closed-form reverse-time adjoint of the surrogate ALIF unroll
 * (functional.py:149-189), with the LIF unroll (functional.py:115-146) as
 * the beta = 0, no-adaptation case.  Forward per step:
 *   m' = m*d + x; th = thr + beta*a; c = k*(m' - th); s = H(c)
 *   m  = m'(1-s) + r s;  a = a*rho + s
 * Reverse, with gm = dL/dm_{t+1}, ga = dL/da_{t+1}:
 *   q   = gs_t + gm*(r - m') + ga          dL/ds_t
 *   gc  = q * k * sigma'(c)                dL/dm' through the spike
 *   gp  = gm*(1-s) + gc                    dL/dm'_t   (= dL/dx_t)
 *   ga <- ga*rho - beta*gc ;  gm <- gp*d
 * gs / gmT / gaT may be NULL (zero).
 */
static void adjoint(const float *x, const float *m0, const float *a0,
                    const float *gs, const float *gmT, const float *gaT,
                    float *gx, float *gm0, float *ga0, int64_t T, int64_t BN,
                    float decay, float rho, float thr, float beta, float reset,
                    float slope, int sid, int alif)
{
    float *pre = (float *)malloc(sizeof(float) * (size_t)T);
    float *th = (float *)malloc(sizeof(float) * (size_t)T);
    for (int64_t i = 0; i < BN; ++i) {
        float m = m0[i], a = alif ? a0[i] : 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            float p = m * decay;
            m = p + x[t * BN + i];
            float tt = alif ? thr + beta * a : thr;
            pre[t] = m;
            th[t] = tt;
            int s = spike_of(m, tt, 1, slope);
            if (s) m = reset;
            if (alif) a = a * rho + (s ? 1.0f : 0.0f);
        }
        float gm = gmT ? gmT[i] : 0.0f;
        float ga = (alif && gaT) ? gaT[i] : 0.0f;
        for (int64_t t = T - 1; t >= 0; --t) {
            float c = slope * (pre[t] - th[t]);
            float s = c >= 0.0f ? 1.0f : 0.0f;
            float dsdm = slope * sg_deriv(sid, c);
            float q = gm * (reset - pre[t]);
            if (gs) q = q + gs[t * BN + i];
            if (alif) q = q + ga;
            float gc = q * dsdm;
            float gp = gm * (1.0f - s) + gc;
            gx[t * BN + i] = gp;
            if (alif) ga = ga * rho - beta * gc;
            gm = gp * decay;
        }
        gm0[i] = gm;
        if (alif) ga0[i] = ga;
    }
    free(pre);
    free(th);
}

void orc_lif_bwd(const float *x, const float *m0, const float *gs,
                 const float *gmT, float *gx, float *gm0, int64_t T,
                 int64_t BN, float decay, float thr, float reset, float slope,
                 int sid)
{
    adjoint(x, m0, NULL, gs, gmT, NULL, gx, gm0, NULL, T, BN, decay, 0.0f, thr,
            0.0f, reset, slope, sid, 0);
}

void orc_alif_bwd(const float *x, const float *m0, const float *a0,
                  const float *gs, const float *gmT, const float *gaT,
                  float *gx, float *gm0, float *ga0, int64_t T, int64_t BN,
                  float decay, float rho, float thr, float beta, float reset,
                  float slope, int sid)
{
    adjoint(x, m0, a0, gs, gmT, gaT, gx, gm0, ga0, T, BN, decay, rho, thr, beta,
            reset, slope, sid, 1);
}

/* pack: bit (n % 32) of word n / 32 is (s[n] != 0); padding bits 0
 * (packing.py:45-71). */
void orc_pack_f32(const float *s, int32_t *words, int64_t rows, int64_t n)
{
    int64_t w = (n + 31) / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < w; ++j) {
            uint32_t v = 0;
            for (int b = 0; b < 32; ++b) {
                int64_t k = j * 32 + b;
                if (k < n && s[r * n + k] != 0.0f) v |= 1u << b;
            }
            words[r * w + j] = (int32_t)v;
        }
}

/* unpack (packing.py:74-81) */
void orc_unpack_f32(const int32_t *words, float *out, int64_t rows, int64_t n)
{
    int64_t w = (n + 31) / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t k = 0; k < n; ++k)
            out[r * n + k] =
                (float)(((uint32_t)words[r * w + k / 32] >> (k % 32)) & 1u);
}

/* per-row popcount with padding masked (packing.py:164-205) */
void orc_row_counts(const int32_t *words, int64_t *counts, int64_t rows, int64_t n)
{
    int64_t w = (n + 31) / 32;
    int rem = (int)(n % 32);
    for (int64_t r = 0; r < rows; ++r) {
        int64_t c = 0;
        for (int64_t j = 0; j < w; ++j) {
            uint32_t v = (uint32_t)words[r * w + j];
            if (j == w - 1 && rem) v &= (1u << rem) - 1u;
            c += __builtin_popcount(v);
        }
        counts[r] = c;
    }
}

/* double-precision sigma'(c) for the exact adjoint below */
static double sg_deriv64(int id, double c)
{
    switch (id) {
    case SG_SIGMOID: {
        double e = exp(-fabs(c)), d = 1.0 + e;
        return e / (d * d);
    }
    case SG_FAST_SIGMOID: {
        double d = 1.0 + fabs(c);
        return 0.5 / (d * d);
    }
    case SG_ATAN: {
        double s = 1.5707963267948966 * c;
        return 0.5 / (1.0 + s * s);
    }
    case SG_TRIANGULAR: {
        double sg = (c > 0.0) ? 1.0 : ((c < 0.0) ? -1.0 : 0.0);
        return fabs(c) < 1.0 ? -sg : 0.0;
    }
    case SG_SUPERSPIKE: {
        double d = 1.0 + fabs(c);
        return 1.0 / (d * d);
    }
    case SG_MULTI_GAUSSIAN: {
        double z = c / 0.5, r = c - 1.0, l = c + 1.0;
        return 0.47873073648171924 * exp(-0.5 * z * z)
             + 0.07978845608028655 * exp(-0.5 * r * r)
             + 0.07978845608028655 * exp(-0.5 * l * l);
    }
    default:
        return 0.0;
    }
}

/*
 * Exact gradient of the fp32 surrogate ALIF forward: the forward runs in
 * fp32 exactly as orc_alif_fwd (so spikes and states are the reference's),
 * the adjoint is evaluated in double along that trajectory.  The centred
 * value c is taken from the fp32 forward so the surrogate branch matches.
 * Outputs are double.  alif = 0 gives the LIF case.
 */
void orc_adjoint_exact(const float *x, const float *m0, const float *a0,
                       const float *gs, const float *gmT, const float *gaT,
                       double *gx, double *gm0, double *ga0, int64_t T,
                       int64_t BN, float decay, float rho, float thr, float beta,
                       float reset, float slope, int sid, int alif)
{
    float *pre = (float *)malloc(sizeof(float) * (size_t)T);
    float *cc = (float *)malloc(sizeof(float) * (size_t)T);
    for (int64_t i = 0; i < BN; ++i) {
        float m = m0[i], a = alif ? a0[i] : 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            float p = m * decay;
            m = p + x[t * BN + i];
            float tt = alif ? thr + beta * a : thr;
            float c = slope * (m - tt);
            pre[t] = m;
            cc[t] = c;
            int s = c >= 0.0f;
            if (s) m = reset;
            if (alif) a = a * rho + (s ? 1.0f : 0.0f);
        }
        double gm = gmT ? (double)gmT[i] : 0.0;
        double ga = (alif && gaT) ? (double)gaT[i] : 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            double s = cc[t] >= 0.0f ? 1.0 : 0.0;
            double q = gm * ((double)reset - (double)pre[t]);
            if (gs) q += (double)gs[t * BN + i];
            if (alif) q += ga;
            double gc = q * (double)slope * sg_deriv64(sid, (double)cc[t]);
            double gp = gm * (1.0 - s) + gc;
            gx[t * BN + i] = gp;
            if (alif) ga = ga * (double)rho - (double)beta * gc;
            gm = gp * (double)decay;
        }
        gm0[i] = gm;
        if (alif) ga0[i] = ga;
    }
    free(pre);
    free(cc);
}

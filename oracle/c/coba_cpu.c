/*
 * CPU restatement of the COBA E/I network step (TEST INFRASTRUCTURE ONLY: the checker and
 * the timed CPU baseline; never linked into the product library).
 *
 * Same algorithm as oracle/neuron.py + oracle/network.py, in C with OpenMP:
 *   - event-driven pre-major scatter over the active rows, the organisation of
 *     brainevent's CPU kernels reached from brainstate/nn/_event_fixedprob.py:205,251;
 *   - the fp32 Expon + COBA + LIFRef update (exp-Euler, brainstate/nn/_exp_euler.py:226-249),
 *     division by the constant tau taken as multiplication by fp32(1/tau) (how XLA runs it);
 *   - its own fp32 exp/exprel (Cody-Waite + degree-7 Taylor, the method the oracle fixes).
 * Built with -ffp-contract=off so every expression is the same rounded op sequence as the
 * numpy oracle; the fused multiply-adds are written out as fmaf (correctly rounded in C99).  Scatter adds use atomics when run multi-threaded: order-free (hence
 * bit-exact) for one repeated weight value, tolerance-equal otherwise.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float o_pow2i(int n) {
  union { uint32_t u; float f; } v;
  v.u = (uint32_t)(n + 127) << 23;
  return v.f;
}

static inline float o_expf(float x) {
  if (x > 88.0f) x = 88.0f;
  if (x < -87.0f) x = -87.0f;
  const float n = nearbyintf(x * (float)1.4426950408889634);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, (float)(0.6931471805599453 - 0.693145751953125), r);
  float p = (float)(1.0 / 5040.0);
  p = fmaf(p, r, (float)(1.0 / 720.0));
  p = fmaf(p, r, (float)(1.0 / 120.0));
  p = fmaf(p, r, (float)(1.0 / 24.0));
  p = fmaf(p, r, (float)(1.0 / 6.0));
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return p * o_pow2i((int)n);
}

static inline float o_exprel(float z) {
  const float az = z < 0.0f ? -z : z;
  if (az < 0.5f) {
    float p = (float)(1.0 / 40320.0);
    p = fmaf(p, z, (float)(1.0 / 5040.0));
    p = fmaf(p, z, (float)(1.0 / 720.0));
    p = fmaf(p, z, (float)(1.0 / 120.0));
    p = fmaf(p, z, (float)(1.0 / 24.0));
    p = fmaf(p, z, (float)(1.0 / 6.0));
    p = fmaf(p, z, 0.5f);
    p = fmaf(p, z, 1.0f);
    return p;
  }
  return (o_expf(z) - 1.0f) / z;
}

typedef struct {
  float V_rest, V_th, V_reset, inv_tau, R, I_ext, E_e, E_i, dt, decay_e, decay_i;
  int32_t ref_steps;
} bso_lif_params;

static inline uint32_t o_mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  x ^= x >> 16;
  return x;
}

int bso_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Runs `steps` steps, the first with absolute index t0.  With a synaptic delay of D steps the
 * inputs form a ring of D+1 slots, in_e/in_i [(D+1) * n]: step t consumes (and clears) slot
 * t mod (D+1), and its spikes are scattered into the same slot, which step t+1+D consumes --
 * an input-side formulation of the spike history the projections read through a Delay.
 * The ring holds the pending inputs before the first step and after the last one.
 * counts/hashes [steps] are written (nullable).  Returns the total number of spikes. */
/* Cloned for CPUs with and without FMA3 (chosen when the library loads): fmaf is one
 * correctly rounded operation either way, in hardware or in the C library. */
__attribute__((target_clones("fma", "default")))
long long bso_coba_lif_run(int n, int n_exc, int k_e, int k_i, const int32_t* idx_e,
                           const float* w_e, float w_e_homo, const int32_t* idx_i,
                           const float* w_i, float w_i_homo, const bso_lif_params* pp,
                           float* V, float* ge, float* gi, int32_t* ref, uint8_t* spk,
                           float* in_e_ring, float* in_i_ring, int steps, int32_t* counts,
                           uint32_t* hashes, int nthreads, int delay, long long t0) {
  const bso_lif_params p = *pp;
  int32_t* active = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
  long long total = 0;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  for (int t = 0; t < steps; ++t) {
    int na = 0;
    uint32_t h = 0;
    const long long slot = (t0 + t) % (long long)(delay + 1);
    float* in_e = in_e_ring + slot * (long long)n;
    float* in_i = in_i_ring + slot * (long long)n;
    /* fused Expon + COBA + LIFRef update; compaction in ascending order */
#pragma omp parallel for schedule(static) reduction(+ : h)
    for (int j = 0; j < n; ++j) {
      float g_e = fmaf(ge[j], p.decay_e, in_e[j]);
      float g_i = fmaf(gi[j], p.decay_i, in_i[j]);
      in_e[j] = 0.0f;
      in_i[j] = 0.0f;
      const float v = V[j];
      float I = fmaf(g_e, p.E_e - v, p.I_ext);
      I = fmaf(g_i, p.E_i - v, I);
      const float f = fmaf(p.R, I, p.V_rest - v) * p.inv_tau;
      const float J = fmaf(-p.R, g_e + g_i, -1.0f) * p.inv_tau;
      const float phi = o_exprel(p.dt * J);
      float vn = fmaf(p.dt * phi, f, v);
      int32_t r = ref[j];
      uint8_t s = 0;
      if (r > 0) {
        vn = v;
        r = r - 1;
      } else if (vn >= p.V_th) {
        s = 1;
        vn = p.V_reset;
        r = p.ref_steps;
      } else {
        r = 0;
      }
      V[j] = vn;
      ge[j] = g_e;
      gi[j] = g_i;
      ref[j] = r;
      spk[j] = s;
      if (s) h += o_mix32((uint32_t)j);
    }
    for (int j = 0; j < n; ++j)
      if (spk[j]) active[na++] = j;
    /* event-driven scatter of this step's spikes into the next step's inputs */
#pragma omp parallel for schedule(dynamic, 4)
    for (int a = 0; a < na; ++a) {
      const int i = active[a];
      if (i < n_exc) {
        const int64_t base = (int64_t)i * k_e;
        for (int k = 0; k < k_e; ++k) {
          const float wv = w_e ? w_e[base + k] : w_e_homo;
          float* o = &in_e[idx_e[base + k]];
#pragma omp atomic
          *o += wv;
        }
      } else {
        const int64_t base = (int64_t)(i - n_exc) * k_i;
        for (int k = 0; k < k_i; ++k) {
          const float wv = w_i ? w_i[base + k] : w_i_homo;
          float* o = &in_i[idx_i[base + k]];
#pragma omp atomic
          *o += wv;
        }
      }
    }
    if (counts) counts[t] = na;
    if (hashes) hashes[t] = h;
    total += na;
  }
  free(active);
  return total;
}

/*
 * CPU restatement of the E/I network step (TEST INFRASTRUCTURE ONLY: the checker and the
 * timed CPU baseline; never linked into the product library).
 *
 * Same algorithm as oracle/neuron.py + oracle/network.py, in C with OpenMP:
 *   - event-driven pre-major scatter over the active rows, the organisation of
 *     brainevent's CPU kernels reached from brainstate/nn/_event_fixedprob.py:205,251;
 *   - the fp32 Expon + COBA/CUBA + LIFRef update (exp-Euler, brainstate/nn/_exp_euler.py:226-249)
 *     or the Expon + COBA + Hodgkin-Huxley update of examples/100_hh_neuron_model.py:49-93,
 *     division by a constant taken as multiplication by its fp32 reciprocal (how XLA runs it);
 *   - its own fp32 exp/exprel (Cody-Waite + degree-7 Taylor, the method the oracle fixes).
 * Built with -ffp-contract=off so every expression is the same rounded op sequence as the
 * numpy oracle; the fused multiply-adds are written out as fmaf (correctly rounded in C99).
 *
 * Input sums of one step (order-free, hence bit-exact under any thread schedule):
 *   - one weight per projection: fp32 atomic adds of that one value, which give w added c
 *     times in one chain whatever the order;
 *   - per-synapse weights: integer sums of the weights rounded to multiples of 2^-S
 *     (S per projection from bso_net_qexp), converted to fp32 once and scaled by 2^-S.
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
  int32_t cuba;
  float scale_e, scale_i;
  int32_t soft_reset;
  int32_t deferred_reset;
} bso_lif_params;

typedef struct {
  float ENa, gNa, EK, gK, EL, gL, inv_C, V_th, I_ext, E_e, E_i, dt, decay_e, decay_i;
} bso_hh_params;

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

static void o_set_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
}

/* ---- fixed-point exponents of per-synapse weights ----
 * For one projection with D = the largest number of its synapses onto one neuron (valid
 * targets) and W = max |w| over its weights, W < 2^e_w (e_w from W's exponent field,
 * -126 for zero or subnormal W) and D <= 2^e_d: S = min(30 - e_w - e_d, 100).  Then every
 * neuron's sum of rint(w * 2^S) stays below 2^31 in magnitude.  Returns 2 if a weight is not
 * finite or S < -100, else 0. */
static int o_qexp_kind(int n, long long nsyn, const int32_t* idx, const float* w, int32_t* S_out) {
  uint32_t wb = 0;
  uint32_t* deg = (uint32_t*)calloc((size_t)(n > 0 ? n : 1), sizeof(uint32_t));
  for (long long s = 0; s < nsyn; ++s) {
    uint32_t b;
    memcpy(&b, &w[s], 4);
    b &= 0x7FFFFFFFu;
    if (b > wb) wb = b;
    const int32_t t = idx[s];
    if (t >= 0 && t < n) ++deg[t];
  }
  uint32_t D = 0;
  for (int j = 0; j < n; ++j)
    if (deg[j] > D) D = deg[j];
  free(deg);
  const int e_w = (wb >> 23) ? (int)(wb >> 23) - 126 : -126;
  int e_d = 0;
  while (((uint64_t)1 << e_d) < D) ++e_d;
  int S = 30 - e_w - e_d;
  if (S > 100) S = 100;
  if (wb >= 0x7F800000u || S < -100) {
    *S_out = 0;
    return 2;
  }
  *S_out = S;
  return 0;
}

int bso_net_qexp(int n, int n_exc, int k_e, int k_i, const int32_t* idx_e, const float* w_e,
                 const int32_t* idx_i, const float* w_i, int32_t* qexp) {
  int e = o_qexp_kind(n, (long long)n_exc * k_e, idx_e, w_e, &qexp[0]);
  int f = o_qexp_kind(n, (long long)(n - n_exc) * k_i, idx_i, w_i, &qexp[1]);
  return e ? e : f;
}

/* ---- one projection's events: the spikes of `active` scattered into the input slot ---- */
typedef struct {
  int n, n_exc, k_e, k_i;
  const int32_t* idx_e;
  const float* w_e;
  float w_e_homo;
  const int32_t* idx_i;
  const float* w_i;
  float w_i_homo;
  float qscale[2], qinv[2];  /* per-synapse weights: 2^S, 2^-S per kind */
} o_net;

static void o_scatter(const o_net* g, const int32_t* active, int na, void* in_e, void* in_i) {
  const int het = g->w_e != NULL;
#pragma omp parallel for schedule(dynamic, 4)
  for (int a = 0; a < na; ++a) {
    const int i = active[a];
    const int inh = i >= g->n_exc;
    const int k = inh ? g->k_i : g->k_e;
    const int64_t base = (int64_t)(inh ? i - g->n_exc : i) * k;
    const int32_t* idx = inh ? g->idx_i : g->idx_e;
    const float* w = inh ? g->w_i : g->w_e;
    void* out = inh ? in_i : in_e;
    for (int s = 0; s < k; ++s) {
      const int32_t t = idx[base + s];
      if (t < 0 || t >= g->n) continue;
      if (het) {
        const int32_t q = (int32_t)nearbyintf(w[base + s] * g->qscale[inh]);
        int32_t* o = &((int32_t*)out)[t];
#pragma omp atomic
        *o += q;
      } else {
        const float wv = inh ? g->w_i_homo : g->w_e_homo;
        float* o = &((float*)out)[t];
#pragma omp atomic
        *o += wv;
      }
    }
  }
}

/* Input of neuron j from a slot, which is cleared (per-synapse weights: int32 sums). */
static inline float o_take(const o_net* g, void* slot, int kind, int j) {
  if (g->w_e != NULL) {
    int32_t* s = (int32_t*)slot;
    const float v = (float)s[j] * g->qinv[kind];
    s[j] = 0;
    return v;
  }
  float* s = (float*)slot;
  const float v = s[j];
  s[j] = 0.0f;
  return v;
}

static void o_net_init(o_net* g, int n, int n_exc, int k_e, int k_i, const int32_t* idx_e,
                       const float* w_e, float w_e_homo, const int32_t* idx_i, const float* w_i,
                       float w_i_homo, const int32_t* qexp) {
  g->n = n;
  g->n_exc = n_exc;
  g->k_e = k_e;
  g->k_i = k_i;
  g->idx_e = idx_e;
  g->w_e = w_e;
  g->w_e_homo = w_e_homo;
  g->idx_i = idx_i;
  g->w_i = w_i;
  g->w_i_homo = w_i_homo;
  for (int k = 0; k < 2; ++k) {
    const int S = qexp ? qexp[k] : 0;
    g->qscale[k] = o_pow2i(S);
    g->qinv[k] = o_pow2i(-S);
  }
}

/* LIFRef + Expon + COBA/CUBA, the operation order of csrc/neuron_dev.h bs_lif_update.
 * deferred_reset: a neuron that spiked in the previous step (prev) is reset first, and a
 * spiking neuron keeps V' (brainpy.state's order). */
static inline float o_lif_reset(const bso_lif_params* p, float v) {
  return p->soft_reset ? v - (p->V_th - p->V_reset) : p->V_reset;
}

static inline uint8_t o_lif(const bso_lif_params* p, float* Vp, float* gep, float* gip,
                            int32_t* refp, float in_e, float in_i, uint8_t prev) {
  const float g_e = fmaf(*gep, p->decay_e, in_e);
  const float g_i = fmaf(*gip, p->decay_i, in_i);
  const float v = (p->deferred_reset && prev) ? o_lif_reset(p, *Vp) : *Vp;
  float I, J;
  if (p->cuba) {
    I = fmaf(g_e, p->scale_e, p->I_ext);
    I = fmaf(g_i, p->scale_i, I);
    J = -1.0f * p->inv_tau;
  } else {
    I = fmaf(g_e, p->E_e - v, p->I_ext);
    I = fmaf(g_i, p->E_i - v, I);
    J = fmaf(-p->R, g_e + g_i, -1.0f) * p->inv_tau;
  }
  const float f = fmaf(p->R, I, p->V_rest - v) * p->inv_tau;
  const float phi = o_exprel(p->dt * J);
  float vn = fmaf(p->dt * phi, f, v);
  int32_t r = *refp;
  uint8_t s = 0;
  if (r > 0) {
    vn = v;
    r = r - 1;
  } else if (vn >= p->V_th) {
    s = 1;
    if (!p->deferred_reset) vn = o_lif_reset(p, vn);
    r = p->ref_steps;
  } else {
    r = 0;
  }
  *Vp = vn;
  *gep = g_e;
  *gip = g_i;
  *refp = r;
  return s;
}

/* Gate exp-Euler step (csrc/neuron_dev.h bs_hh_gate). */
static inline float o_gate(float x, float a, float b, float dt) {
  const float f = fmaf(a, 1.0f - x, -(b * x));
  const float J = -(a + b);
  const float phi = o_exprel(dt * J);
  return fmaf(dt * phi, f, x);
}

/* Expon + COBA + HH (csrc/neuron_dev.h bs_hh_prepare + bs_hh_finish). */
static inline uint8_t o_hh(const bso_hh_params* p, float* Vp, float* mp, float* hp, float* np_,
                           float* gep, float* gip, float in_e, float in_i) {
  const float V = *Vp, m = *mp, h = *hp, n = *np_;
  const float k10 = 1.0f / 10.0f, k18 = 1.0f / 18.0f, k20 = 1.0f / 20.0f, k80 = 1.0f / 80.0f;
  const float am = 1.0f / o_exprel((-(V + 40.0f)) * k10);
  const float bm = 4.0f * o_expf((-(V + 65.0f)) * k18);
  const float ah = 0.07f * o_expf((-(V + 65.0f)) * k20);
  const float bh = 1.0f / (1.0f + o_expf((-(V + 35.0f)) * k10));
  const float an = 0.1f / o_exprel((-(V + 55.0f)) * k10);
  const float bn = 0.125f * o_expf((-(V + 65.0f)) * k80);
  const float gna = p->gNa * m * m * m * h;
  const float n2 = n * n;
  const float gk = p->gK * n2 * n2;
  const float mn = o_gate(m, am, bm, p->dt);
  const float hn = o_gate(h, ah, bh, p->dt);
  const float nn = o_gate(n, an, bn, p->dt);
  const float ge = fmaf(*gep, p->decay_e, in_e);
  const float gi = fmaf(*gip, p->decay_i, in_i);
  float I = fmaf(ge, p->E_e - V, p->I_ext);
  I = fmaf(gi, p->E_i - V, I);
  float acc = fmaf(-gna, V - p->ENa, I);
  acc = fmaf(-gk, V - p->EK, acc);
  acc = fmaf(-p->gL, V - p->EL, acc);
  const float f = acc * p->inv_C;
  const float J = ((((-gna) - gk) - p->gL) - (ge + gi)) * p->inv_C;
  const float phi = o_exprel(p->dt * J);
  const float Vn = fmaf(p->dt * phi, f, V);
  *Vp = Vn;
  *mp = mn;
  *hp = hn;
  *np_ = nn;
  *gep = ge;
  *gip = gi;
  return (V < p->V_th) && (Vn >= p->V_th);
}

/* Runs `steps` steps, the first with absolute index t0.  With a synaptic delay of D steps the
 * inputs form a ring of D+1 slots, in_e/in_i [(D+1) * n] (float, or int32 fixed-point sums with
 * per-synapse weights): step t consumes (and clears) slot t mod (D+1), and its spikes are
 * scattered into the same slot, which step t+1+D consumes -- an input-side formulation of the
 * spike history the projections read through a Delay.  The ring holds the pending inputs
 * before the first step and after the last one.  counts/hashes [steps] are written
 * (nullable).  model 0: LIF (st = V, ge, gi, ref), 1: HH (st = V, m, h, n, ge, gi).
 * Returns the total number of spikes. */
static long long o_run(int model, const o_net* g, const void* params, void* const* st,
                       uint8_t* spk, void* in_e_ring, void* in_i_ring, int steps,
                       int32_t* counts, uint32_t* hashes, int nthreads, int delay,
                       long long t0, const float* iext) {
  const int n = g->n;
  int32_t* active = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
  long long total = 0;
  o_set_threads(nthreads);
  for (int t = 0; t < steps; ++t) {
    int na = 0;
    uint32_t h = 0;
    const long long slot = (t0 + t) % (long long)(delay + 1);
    char* in_e = (char*)in_e_ring + slot * (long long)n * 4;
    char* in_i = (char*)in_i_ring + slot * (long long)n * 4;
    if (model == 0) {
      const bso_lif_params* p = (const bso_lif_params*)params;
      float* V = (float*)st[0];
      float* ge = (float*)st[1];
      float* gi = (float*)st[2];
      int32_t* ref = (int32_t*)st[3];
#pragma omp parallel for schedule(static) reduction(+ : h)
      for (int j = 0; j < n; ++j) {
        const float ie = o_take(g, in_e, 0, j), ii = o_take(g, in_i, 1, j);
        bso_lif_params q = *p;
        if (iext) q.I_ext = iext[j];  /* per-neuron external input */
        const uint8_t s = o_lif(&q, &V[j], &ge[j], &gi[j], &ref[j], ie, ii, spk[j]);
        spk[j] = s;
        if (s) h += o_mix32((uint32_t)j);
      }
    } else {
      const bso_hh_params* p = (const bso_hh_params*)params;
      float* V = (float*)st[0];
      float* m = (float*)st[1];
      float* hg = (float*)st[2];
      float* ng = (float*)st[3];
      float* ge = (float*)st[4];
      float* gi = (float*)st[5];
#pragma omp parallel for schedule(static) reduction(+ : h)
      for (int j = 0; j < n; ++j) {
        const float ie = o_take(g, in_e, 0, j), ii = o_take(g, in_i, 1, j);
        bso_hh_params q = *p;
        if (iext) q.I_ext = iext[j];
        const uint8_t s = o_hh(&q, &V[j], &m[j], &hg[j], &ng[j], &ge[j], &gi[j], ie, ii);
        spk[j] = s;
        if (s) h += o_mix32((uint32_t)j);
      }
    }
    for (int j = 0; j < n; ++j)
      if (spk[j]) active[na++] = j;
    o_scatter(g, active, na, in_e, in_i);
    if (counts) counts[t] = na;
    if (hashes) hashes[t] = h;
    total += na;
  }
  free(active);
  return total;
}

/* Cloned for CPUs with and without FMA3 (chosen when the library loads): fmaf is one
 * correctly rounded operation either way, in hardware or in the C library.  `qexp` [2] is
 * bso_net_qexp's result (per-synapse weights; ignored otherwise). */
__attribute__((target_clones("fma", "default")))
long long bso_coba_lif_run(int n, int n_exc, int k_e, int k_i, const int32_t* idx_e,
                           const float* w_e, float w_e_homo, const int32_t* idx_i,
                           const float* w_i, float w_i_homo, const bso_lif_params* pp,
                           float* V, float* ge, float* gi, int32_t* ref, uint8_t* spk,
                           void* in_e_ring, void* in_i_ring, int steps, int32_t* counts,
                           uint32_t* hashes, int nthreads, int delay, long long t0,
                           const int32_t* qexp, const float* iext) {
  o_net g;
  o_net_init(&g, n, n_exc, k_e, k_i, idx_e, w_e, w_e_homo, idx_i, w_i, w_i_homo, qexp);
  void* st[4] = {V, ge, gi, ref};
  return o_run(0, &g, pp, st, spk, in_e_ring, in_i_ring, steps, counts, hashes, nthreads, delay,
               t0, iext);
}

__attribute__((target_clones("fma", "default")))
long long bso_coba_hh_run(int n, int n_exc, int k_e, int k_i, const int32_t* idx_e,
                          const float* w_e, float w_e_homo, const int32_t* idx_i,
                          const float* w_i, float w_i_homo, const bso_hh_params* pp, float* V,
                          float* m, float* h, float* ng, float* ge, float* gi, uint8_t* spk,
                          void* in_e_ring, void* in_i_ring, int steps, int32_t* counts,
                          uint32_t* hashes, int nthreads, int delay, long long t0,
                          const int32_t* qexp, const float* iext) {
  o_net g;
  o_net_init(&g, n, n_exc, k_e, k_i, idx_e, w_e, w_e_homo, idx_i, w_i, w_i_homo, qexp);
  void* st[6] = {V, m, h, ng, ge, gi};
  return o_run(1, &g, pp, st, spk, in_e_ring, in_i_ring, steps, counts, hashes, nthreads, delay,
               t0, iext);
}

/* Steady-state gates x_inf = a / (a + b) at V (examples/100_hh_neuron_model.py:66-70). */
__attribute__((target_clones("fma", "default")))
void bso_hh_init(int n, const float* V, float* m, float* h, float* ng) {
  const float k10 = 1.0f / 10.0f, k18 = 1.0f / 18.0f, k20 = 1.0f / 20.0f, k80 = 1.0f / 80.0f;
  for (int j = 0; j < n; ++j) {
    const float v = V[j];
    const float am = 1.0f / o_exprel((-(v + 40.0f)) * k10);
    const float bm = 4.0f * o_expf((-(v + 65.0f)) * k18);
    const float ah = 0.07f * o_expf((-(v + 65.0f)) * k20);
    const float bh = 1.0f / (1.0f + o_expf((-(v + 35.0f)) * k10));
    const float an = 0.1f / o_exprel((-(v + 55.0f)) * k10);
    const float bn = 0.125f * o_expf((-(v + 65.0f)) * k80);
    m[j] = am / (am + bm);
    h[j] = ah / (ah + bh);
    ng[j] = an / (an + bn);
  }
}

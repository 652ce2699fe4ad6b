// Per-neuron fused updates (device side), shared by the single-step kernels and the
// persistent network runners.  Every expression follows the operation order of the
// reference code, with each multiply-add written as one fused multiply-add (bs_fma), and
// the library is built with -ffp-contract=off, so each line is a fixed sequence of
// correctly rounded fp32 operations that the CPU restatements reproduce bit for bit.
// Division by a model constant (tau, C, the HH rate scales) is multiplication by its fp32
// reciprocal: that is how the reference executes it under jit, where XLA's algebraic
// simplifier rewrites A / Const into A * (1 / Const).  Divisions by variables stay divisions.
#pragma once

#include "bs_math.h"
#include "common.h"

// V after a spike: V_reset (hard reset) or V' - (V_th - V_reset) (kSoft: subtractive).
template <bool kSoft>
__device__ __forceinline__ float bs_lif_reset(const bs_lif_params& p, float v) {
  return kSoft ? v - (p.V_th - p.V_reset) : p.V_reset;
}

// The exp-Euler membrane step V -> V' given the conductances after this step's update
// (everything of bs_lif_update that V' depends on: V, ge', gi' and the parameters).  The CUBA
// current does not depend on V, so the exp-Euler Jacobian is -1 * inv_tau.
template <bool kCuba>
__device__ __forceinline__ float bs_lif_vnext(const bs_lif_params& p, float V, float ge,
                                              float gi) {
  float I, J;
  if constexpr (kCuba) {
    I = bs_fma(ge, p.scale_e, p.I_ext);
    I = bs_fma(gi, p.scale_i, I);
    J = -1.0f * p.inv_tau;
  } else {
    I = bs_fma(ge, p.E_e - V, p.I_ext);
    I = bs_fma(gi, p.E_i - V, I);
    J = bs_fma(-p.R, ge + gi, -1.0f) * p.inv_tau;
  }
  const float f = bs_fma(p.R, I, p.V_rest - V) * p.inv_tau;
  const float phi = bs_exprel(p.dt * J);
  return bs_fma(p.dt * phi, f, V);
}

// brainpy.state Expon + COBA (kCuba: CUBA) + LIFRef for one neuron; see bs_lif_params in the
// header.  Returns the spike; updates V, ge, gi, ref in place.  kSoft: a spike subtracts
// V_th - V_reset from V' (p.soft_reset) instead of setting V_reset.  kKeep: a spiking neuron
// keeps V' (the reset is left to the start of its next step, p.deferred_reset).  All are
// compile-time choices so that the persistent runner's update carries no per-neuron selects.
template <bool kCuba = false, bool kSoft = false, bool kKeep = false>
__device__ __forceinline__ bool bs_lif_update(const bs_lif_params& p, float& V, float& ge,
                                              float& gi, int32_t& ref, float in_e, float in_i) {
  ge = bs_fma(ge, p.decay_e, in_e);
  gi = bs_fma(gi, p.decay_i, in_i);
  float Vn = bs_lif_vnext<kCuba>(p, V, ge, gi);
  bool spk = false;
  if (ref > 0) {
    Vn = V;
    ref = ref - 1;
  } else {
    spk = Vn >= p.V_th;
    if (spk) {
      if (!kKeep) Vn = bs_lif_reset<kSoft>(p, Vn);
      ref = p.ref_steps;
    } else {
      ref = 0;
    }
  }
  V = Vn;
  return spk;
}

// bs_lif_update with the output kind and reset taken from p at run time (uniform branch).
__device__ __forceinline__ bool bs_lif_update_p(const bs_lif_params& p, float& V, float& ge,
                                                float& gi, int32_t& ref, float in_e,
                                                float in_i) {
  if (p.cuba)
    return p.soft_reset ? bs_lif_update<true, true>(p, V, ge, gi, ref, in_e, in_i)
                        : bs_lif_update<true, false>(p, V, ge, gi, ref, in_e, in_i);
  return p.soft_reset ? bs_lif_update<false, true>(p, V, ge, gi, ref, in_e, in_i)
                      : bs_lif_update<false, false>(p, V, ge, gi, ref, in_e, in_i);
}

struct bs_hh_rates {
  float am, bm, ah, bh, an, bn;
};

// examples/100_hh_neuron_model.py:49-64 (V in mV, rates in 1/ms).
__device__ __forceinline__ bs_hh_rates bs_hh_rate(float V) {
  bs_hh_rates r;
  constexpr float k10 = 1.0f / 10.0f, k18 = 1.0f / 18.0f;  // fp32 reciprocals
  constexpr float k20 = 1.0f / 20.0f, k80 = 1.0f / 80.0f;
  r.am = 1.0f / bs_exprel((-(V + 40.0f)) * k10);
  r.bm = 4.0f * bs_expf((-(V + 65.0f)) * k18);
  r.ah = 0.07f * bs_expf((-(V + 65.0f)) * k20);
  r.bh = 1.0f / (1.0f + bs_expf((-(V + 35.0f)) * k10));
  r.an = 0.1f / bs_exprel((-(V + 55.0f)) * k10);
  r.bn = 0.125f * bs_expf((-(V + 65.0f)) * k80);
  return r;
}

__device__ __forceinline__ float bs_hh_gate(float x, float a, float b, float dt) {
  const float f = bs_fma(a, 1.0f - x, -(b * x));
  const float J = -(a + b);
  const float phi = bs_exprel(dt * J);
  return bs_fma(dt * phi, f, x);
}

// The part of one HH step that does not depend on this step's synaptic input: the gate
// updates (rates of the previous V, exp-Euler per gate) and the channel conductances of the
// previous m, h, n.  Same operations as inline, so splitting the step changes no bit.
struct bs_hh_pre {
  float mn, hn, nn;  // gates after the step
  float gna, gk;     // gNa m^3 h and gK n^4 of the previous gates
};

__device__ __forceinline__ bs_hh_pre bs_hh_prepare(const bs_hh_params& p, float V, float m,
                                                   float h, float n) {
  const bs_hh_rates r = bs_hh_rate(V);
  bs_hh_pre q;
  q.gna = p.gNa * m * m * m * h;
  const float n2 = n * n;
  q.gk = p.gK * n2 * n2;
  q.mn = bs_hh_gate(m, r.am, r.bm, p.dt);
  q.hn = bs_hh_gate(h, r.ah, r.bh, p.dt);
  q.nn = bs_hh_gate(n, r.an, r.bn, p.dt);
  return q;
}

// The rest of the step: Expon + COBA conductances from this step's input and the
// exp-Euler step of V (examples/100_hh_neuron_model.py:72-93).
__device__ __forceinline__ bool bs_hh_finish(const bs_hh_params& p, const bs_hh_pre& q, float& V,
                                             float& m, float& h, float& n, float& ge,
                                             float& gi, float in_e, float in_i) {
  ge = bs_fma(ge, p.decay_e, in_e);
  gi = bs_fma(gi, p.decay_i, in_i);
  float I = bs_fma(ge, p.E_e - V, p.I_ext);
  I = bs_fma(gi, p.E_i - V, I);
  // (I - INa - IK - IL) / C, each channel current folded in with one fused multiply-add
  float acc = bs_fma(-q.gna, V - p.ENa, I);
  acc = bs_fma(-q.gk, V - p.EK, acc);
  acc = bs_fma(-p.gL, V - p.EL, acc);
  const float f = acc * p.inv_C;
  const float J = ((((-q.gna) - q.gk) - p.gL) - (ge + gi)) * p.inv_C;
  const float phi = bs_exprel(p.dt * J);
  const float Vn = bs_fma(p.dt * phi, f, V);
  const bool spk = (V < p.V_th) && (Vn >= p.V_th);
  V = Vn;
  m = q.mn;
  h = q.hn;
  n = q.nn;
  return spk;
}

// Expon + COBA + HH exp-Euler for one neuron (examples/100_hh_neuron_model.py:72-93).
__device__ __forceinline__ bool bs_hh_update(const bs_hh_params& p, float& V, float& m, float& h,
                                             float& n, float& ge, float& gi, float in_e,
                                             float in_i) {
  const bs_hh_pre q = bs_hh_prepare(p, V, m, h, n);
  return bs_hh_finish(p, q, V, m, h, n, ge, gi, in_e, in_i);
}

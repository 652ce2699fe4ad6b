// N3: fused neuron + synapse state updates, one thread per neuron.
//
// Each neuron's state is read once and written once per step (LIF: V, g_e, g_i, ref and
// the spike byte; HH: V, m, h, n, g_e, g_i and the spike byte).  Pure streaming: the
// bound is HBM bandwidth.
#include "neuron_dev.h"

namespace {

constexpr int kBlock = 256;

template <bool kCuba, bool kSoft>
__global__ __launch_bounds__(kBlock) void k_lif_step(int32_t n, float* __restrict__ V,
                                                     float* __restrict__ ge,
                                                     float* __restrict__ gi,
                                                     int32_t* __restrict__ ref,
                                                     const float* __restrict__ in_e,
                                                     const float* __restrict__ in_i,
                                                     const float* __restrict__ iext,
                                                     bs_lif_arrays pa, bs_lif_params p,
                                                     uint8_t* __restrict__ spk) {
  for (int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x; j < n;
       j += (int64_t)gridDim.x * kBlock) {
    float v = V[j], e = ge[j], i = gi[j];
    int32_t r = ref[j];
    bs_lif_params q = p;
    if (iext) q.I_ext = iext[j];  // per-neuron external input
    // per-neuron parameters (uniform branches: each array is given or not)
    if (pa.V_rest) q.V_rest = pa.V_rest[j];
    if (pa.V_th) q.V_th = pa.V_th[j];
    if (pa.V_reset) q.V_reset = pa.V_reset[j];
    if (pa.inv_tau) q.inv_tau = pa.inv_tau[j];
    if (pa.R) q.R = pa.R[j];
    if (pa.ref_steps) q.ref_steps = pa.ref_steps[j];
    const float xe = in_e ? in_e[j] : 0.0f, xi = in_i ? in_i[j] : 0.0f;
    bool s;
    if (p.deferred_reset) {  // spk holds the previous step's spikes: their reset comes first
      if (spk[j]) v = bs_lif_reset<kSoft>(q, v);
      s = bs_lif_update<kCuba, kSoft, true>(q, v, e, i, r, xe, xi);
    } else {
      s = bs_lif_update<kCuba, kSoft, false>(q, v, e, i, r, xe, xi);
    }
    V[j] = v;
    ge[j] = e;
    gi[j] = i;
    ref[j] = r;
    if (spk) spk[j] = s ? 1 : 0;
  }
}

__global__ __launch_bounds__(kBlock) void k_hh_init(int32_t n, const float* __restrict__ V,
                                                    float* __restrict__ m, float* __restrict__ h,
                                                    float* __restrict__ ng) {
  for (int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x; j < n;
       j += (int64_t)gridDim.x * kBlock) {
    const bs_hh_rates r = bs_hh_rate(V[j]);
    m[j] = r.am / (r.am + r.bm);
    h[j] = r.ah / (r.ah + r.bh);
    ng[j] = r.an / (r.an + r.bn);
  }
}

__global__ __launch_bounds__(kBlock) void k_hh_step(int32_t n, float* __restrict__ V,
                                                    float* __restrict__ m, float* __restrict__ h,
                                                    float* __restrict__ ng,
                                                    float* __restrict__ ge,
                                                    float* __restrict__ gi,
                                                    const float* __restrict__ in_e,
                                                    const float* __restrict__ in_i,
                                                    const float* __restrict__ iext,
                                                    bs_hh_arrays pa, bs_hh_params p,
                                                    uint8_t* __restrict__ spk) {
  for (int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x; j < n;
       j += (int64_t)gridDim.x * kBlock) {
    float v = V[j], mm = m[j], hh = h[j], nn = ng[j], e = ge[j], i = gi[j];
    bs_hh_params q = p;
    if (iext) q.I_ext = iext[j];
    if (pa.ENa) q.ENa = pa.ENa[j];  // per-neuron parameters (uniform branches)
    if (pa.gNa) q.gNa = pa.gNa[j];
    if (pa.EK) q.EK = pa.EK[j];
    if (pa.gK) q.gK = pa.gK[j];
    if (pa.EL) q.EL = pa.EL[j];
    if (pa.gL) q.gL = pa.gL[j];
    if (pa.inv_C) q.inv_C = pa.inv_C[j];
    if (pa.V_th) q.V_th = pa.V_th[j];  // per-neuron external input
    const bool s = bs_hh_update(q, v, mm, hh, nn, e, i, in_e ? in_e[j] : 0.0f,
                                in_i ? in_i[j] : 0.0f);
    V[j] = v;
    m[j] = mm;
    h[j] = hh;
    ng[j] = nn;
    ge[j] = e;
    gi[j] = i;
    if (spk) spk[j] = s ? 1 : 0;
  }
}

// Exponential Euler of a general drift (brainstate/nn/_exp_euler.py:226-249):
//   out = x + (dt * exprel(dt * J)) * f,  one fused multiply-add, as the fused updates write
// it, so a drift and Jacobian that equal theirs give their bits.
__global__ __launch_bounds__(kBlock) void k_exp_euler_f32(int64_t n, const float* __restrict__ x,
                                                         const float* __restrict__ f,
                                                         const float* __restrict__ jac, float dt,
                                                         float* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock) {
    const float phi = bs_exprel(dt * jac[i]);
    out[i] = bs_fma(dt * phi, f[i], x[i]);
  }
}

// Double-precision exprel: series below 1e-3 (truncation < 1e-13 relative), expm1(z) / z
// elsewhere.
__device__ __forceinline__ double exprel_f64(double z) {
  if (fabs(z) < 1e-3) return 1.0 + z * (0.5 + z * (1.0 / 6.0 + z * (1.0 / 24.0 + z / 120.0)));
  return expm1(z) / z;
}

__global__ __launch_bounds__(kBlock) void k_exp_euler_f64(int64_t n, const double* __restrict__ x,
                                                         const double* __restrict__ f,
                                                         const double* __restrict__ jac,
                                                         double dt, double* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock) {
    const double phi = exprel_f64(dt * jac[i]);
    out[i] = fma(dt * phi, f[i], x[i]);
  }
}

int grid(int32_t n) {
  int64_t b = ((int64_t)n + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)bs_num_cus() * 16;
  return (int)(b < 1 ? 1 : (b > cap ? cap : b));
}

}  // namespace

extern "C" int bs_coba_lif_step_arr(int32_t n, float* V, float* ge, float* gi, int32_t* ref,
                                    const float* in_e, const float* in_i, const float* I_ext,
                                    const bs_lif_arrays* arr, const bs_lif_params* p,
                                    uint8_t* spk_out, bs_stream_t stream) {
  const bs_lif_arrays pa = arr ? *arr : bs_lif_arrays{};
  bs_clear_error();
  BS_CHECK_ARG(n >= 0, "bs_coba_lif_step: n=%d < 0", n);
  BS_CHECK_ARG(p != nullptr, "bs_coba_lif_step: params are NULL");
  BS_CHECK_ARG(p->inv_tau == p->inv_tau, "bs_coba_lif_step: inv_tau is NaN");
  if (n == 0) return BS_OK;
  BS_CHECK_ARG(V && ge && gi && ref, "bs_coba_lif_step: NULL state pointer");
  BS_CHECK_ARG(!p->deferred_reset || spk_out != nullptr,
               "bs_coba_lif_step: deferred_reset reads the previous spikes from spk_out, "
               "which is NULL");
  hipStream_t s = bs_stream(stream);
#define BS_LIF(C, S) \
  k_lif_step<C, S><<<grid(n), kBlock, 0, s>>>(n, V, ge, gi, ref, in_e, in_i, I_ext, pa, *p, \
                                              spk_out)
  if (p->cuba) { if (p->soft_reset) BS_LIF(true, true); else BS_LIF(true, false); }
  else { if (p->soft_reset) BS_LIF(false, true); else BS_LIF(false, false); }
#undef BS_LIF
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_coba_lif_step_in(int32_t n, float* V, float* ge, float* gi, int32_t* ref,
                                   const float* in_e, const float* in_i, const float* I_ext,
                                   const bs_lif_params* p, uint8_t* spk_out,
                                   bs_stream_t stream) {
  return bs_coba_lif_step_arr(n, V, ge, gi, ref, in_e, in_i, I_ext, nullptr, p, spk_out, stream);
}

extern "C" int bs_coba_lif_step(int32_t n, float* V, float* ge, float* gi, int32_t* ref,
                                const float* in_e, const float* in_i, const bs_lif_params* p,
                                uint8_t* spk_out, bs_stream_t stream) {
  return bs_coba_lif_step_arr(n, V, ge, gi, ref, in_e, in_i, nullptr, nullptr, p, spk_out,
                              stream);
}

extern "C" int bs_hh_init(int32_t n, const float* V, float* m, float* h, float* ng,
                          bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n >= 0, "bs_hh_init: n=%d < 0", n);
  if (n == 0) return BS_OK;
  BS_CHECK_ARG(V && m && h && ng, "bs_hh_init: NULL pointer");
  k_hh_init<<<grid(n), kBlock, 0, bs_stream(stream)>>>(n, V, m, h, ng);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_coba_hh_step_arr(int32_t n, float* V, float* m, float* h, float* ng,
                                   float* ge, float* gi, const float* in_e, const float* in_i,
                                   const float* I_ext, const bs_hh_arrays* arr,
                                   const bs_hh_params* p, uint8_t* spk_out, bs_stream_t stream) {
  const bs_hh_arrays pa = arr ? *arr : bs_hh_arrays{};
  bs_clear_error();
  BS_CHECK_ARG(n >= 0, "bs_coba_hh_step: n=%d < 0", n);
  BS_CHECK_ARG(p != nullptr, "bs_coba_hh_step: params are NULL");
  BS_CHECK_ARG(p->inv_C == p->inv_C, "bs_coba_hh_step: inv_C is NaN");
  if (n == 0) return BS_OK;
  BS_CHECK_ARG(V && m && h && ng && ge && gi, "bs_coba_hh_step: NULL state pointer");
  k_hh_step<<<grid(n), kBlock, 0, bs_stream(stream)>>>(n, V, m, h, ng, ge, gi, in_e, in_i,
                                                        I_ext, pa, *p, spk_out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_coba_hh_step_in(int32_t n, float* V, float* m, float* h, float* ng, float* ge,
                                  float* gi, const float* in_e, const float* in_i,
                                  const float* I_ext, const bs_hh_params* p, uint8_t* spk_out,
                                  bs_stream_t stream) {
  return bs_coba_hh_step_arr(n, V, m, h, ng, ge, gi, in_e, in_i, I_ext, nullptr, p, spk_out,
                             stream);
}

extern "C" int bs_coba_hh_step(int32_t n, float* V, float* m, float* h, float* ng, float* ge,
                               float* gi, const float* in_e, const float* in_i,
                               const bs_hh_params* p, uint8_t* spk_out, bs_stream_t stream) {
  return bs_coba_hh_step_arr(n, V, m, h, ng, ge, gi, in_e, in_i, nullptr, nullptr, p, spk_out,
                             stream);
}

extern "C" int bs_exp_euler_f32(int64_t n, const float* x, const float* drift, const float* jac,
                                float dt, float* out, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n >= 0 && n < ((int64_t)1 << 40), "bs_exp_euler_f32: n=%lld out of range",
               (long long)n);
  if (n == 0) return BS_OK;
  BS_CHECK_ARG(x && drift && jac && out, "bs_exp_euler_f32: NULL pointer");
  const int g = grid((int32_t)(n < (1 << 30) ? n : (1 << 30)));
  k_exp_euler_f32<<<g, kBlock, 0, bs_stream(stream)>>>(n, x, drift, jac, dt, out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_exp_euler_f64(int64_t n, const double* x, const double* drift,
                                const double* jac, double dt, double* out, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n >= 0 && n < ((int64_t)1 << 40), "bs_exp_euler_f64: n=%lld out of range",
               (long long)n);
  if (n == 0) return BS_OK;
  BS_CHECK_ARG(x && drift && jac && out, "bs_exp_euler_f64: NULL pointer");
  const int g = grid((int32_t)(n < (1 << 30) ? n : (1 << 30)));
  k_exp_euler_f64<<<g, kBlock, 0, bs_stream(stream)>>>(n, x, drift, jac, dt, out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

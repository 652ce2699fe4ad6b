/*
 * brainstate_amd -- C ABI of the MI355X (gfx950) engine for brainstate's spiking-network step.
 *
 * Plain C types only: device pointers, sizes, a stream handle and int status codes.
 * All array pointers are device memory owned by the caller; the library never frees
 * caller memory and keeps no pointer across calls.  Work is enqueued on the given
 * stream (a hipStream_t passed as void*; NULL = the null stream) with no host
 * synchronisation.  A nonzero status comes with a thread-local message from
 * bs_last_error().
 *
 * Each entry point names the reference interface it replaces (file:line under the
 * chaobrain/brainstate 0.5.4 tree).  The arithmetic of those interfaces lives in the
 * un-vendored dependencies brainevent (event operators) and brainpy.state (neuron and
 * synapse models); the reference reaches them at the cited call sites.
 */
#ifndef BRAINSTATE_AMD_H_
#define BRAINSTATE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define BS_API __attribute__((visibility("default")))
#else
#define BS_API
#endif

typedef void* bs_stream_t;

enum bs_status {
  BS_OK = 0,
  BS_ERR_INVALID = 1,     /* bad shape, dtype, pointer or parameter */
  BS_ERR_LAUNCH = 2,      /* HIP runtime / launch failure */
  BS_ERR_UNSUPPORTED = 3  /* e.g. the device cannot co-schedule a persistent grid */
};

/* Spike vector element types accepted by the event operators: nonzero = one event
 * (brainevent.EventArray semantics, brainstate/nn/_event_fixedprob.py:249-252). */
enum bs_spike_dtype { BS_SPK_U8 = 0, BS_SPK_F32 = 1 };

BS_API const char* bs_last_error(void);
BS_API int bs_version(void);

/* ---------------------------------------------------------------- N1 spike compaction
 * Replaces the zero-skipping inside brainevent's event kernels (no reference symbol;
 * the spikes reach it from brainstate/nn/_event_fixedprob.py:251).
 * idx_out[0..count) = ascending indices i with spk[i] != 0; *count_out = count.
 * `workspace` holds bs_spike_compact_workspace_size(n) bytes, zero-filled once when
 * allocated; each call leaves it ready for the next.  Calls that share a workspace
 * must be ordered on one stream. n < 2^30. */
BS_API size_t bs_spike_compact_workspace_size(int32_t n);
BS_API int bs_spike_compact(const void* spk, int32_t spk_dtype, int32_t n, int32_t* idx_out,
                     int32_t* count_out, void* workspace, bs_stream_t stream);

/* bs_spike_compact without a workspace and without allocating: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The scan state lives in a static
 * device array of 33,024 bytes that each device holds until the process ends, so
 * n <= 67,108,864 (larger n: BS_ERR_INVALID; use bs_spike_compact).  The first call on a
 * device clears that array with a kernel on `stream`; every call leaves it ready for the
 * next.  All calls on one device share the array: calls that overlap in time on one device
 * (different streams or threads without ordering) race and give wrong results. */
BS_API int bs_spike_compact_noalloc(const void* spk, int32_t spk_dtype, int32_t n,
                                    int32_t* idx_out, int32_t* count_out, bs_stream_t stream);

/* ---------------------------------------------------------------- N2a event scatter
 * Replaces `EventArray(spk) @ FixedPostNumConn((w, idx))` and `... @ CSR((w, idx, indptr))`
 * (brainstate/nn/_event_fixedprob.py:176-181,192,202-205,249-252).
 * For each active pre row r = active[a], a < *n_active, adds w of each synapse of r to
 * out[target].  Rows: fixed-num (indptr == NULL) -> synapses r*k .. r*k+k-1; CSR ->
 * indptr[r] .. indptr[r+1]-1 (nnz = indptr[n_pre]).  w == NULL -> homogeneous w_homo.
 * accumulate == 0 zero-fills out[n_post] first.  fp32 atomics: the order of additions
 * is unspecified (sums of one repeated weight value are order-free and exact).
 * Out-of-range rows / targets are skipped. */
BS_API int bs_event_scatter_f32(const int32_t* active, const int32_t* n_active, int32_t n_pre,
                         const int32_t* indptr, const int32_t* indices, int32_t k,
                         const float* w, float w_homo, int32_t n_post, float* out,
                         int32_t accumulate, bs_stream_t stream);

/* Same operator taking the spike vector directly (nonzero = event): one launch compacts and
 * scatters (plus a zero-fill unless accumulate).  With per-synapse weights, a workgroup
 * holding >= 4 events per output aggregates them in LDS first when n_post <= 16384. */
BS_API int bs_event_matvec_f32(const void* spk, int32_t spk_dtype, int32_t n_pre,
                               const int32_t* indptr, const int32_t* indices, int32_t k,
                               const float* w, float w_homo, int32_t n_post, float* out,
                               int32_t accumulate, bs_stream_t stream);

/* Value-weighted form of the same operator: out[j] (+)= sum_{i,k: idx[i,k]=j} x[i] * w[i,k]
 * for fp32 x (rows with x[i] == 0 are skipped).  Used for the forward-mode derivative of the
 * event mat-vec: d(out) = value_matvec(dx, w) + value_matvec(x, dw).  No counterpart call in
 * brainstate itself; replaces the tangent rule of brainevent's event mat-vec primitive, whose
 * numerics the reference pins at brainstate/nn/_event_fixedprob_test.py:90-126. */
BS_API int bs_value_matvec_f32(const float* x, int32_t n_pre, const int32_t* indptr,
                               const int32_t* indices, int32_t k, const float* w, float w_homo,
                               int32_t n_post, float* out, int32_t accumulate,
                               bs_stream_t stream);

/* Batched forms: `batch` spike / value rows [batch, n_pre] against one connectivity, outputs
 * [batch, n_post], one launch.  Replaces `EventArray(spk) @ conn` with a leading batch
 * dimension (brainstate/nn/_event_fixedprob.py:202-209 under init_all_states(batch_size),
 * and vmap2 over replicas, brainstate/transform/_mapping2.py:289).  batch <= 65535. */
BS_API int bs_event_matvec_batch_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                     int32_t n_pre, const int32_t* indptr, const int32_t* indices,
                                     int32_t k, const float* w, float w_homo, int32_t n_post,
                                     float* out, int32_t accumulate, bs_stream_t stream);
BS_API int bs_value_matvec_batch_f32(const float* x, int32_t batch, int32_t n_pre,
                                     const int32_t* indptr, const int32_t* indices, int32_t k,
                                     const float* w, float w_homo, int32_t n_post, float* out,
                                     int32_t accumulate, bs_stream_t stream);

/* Reverse mode of the event mat-vec (the VJP the reference checks at
 * brainstate/nn/_event_fixedprob_test.py:56-88): with g = grad_out[n_post] and x[i] the spike
 * value (0/1 for byte spikes),
 *   grad_spk[i] = sum_k w[i,k] * g[idx[i,k]]                      (nullable, [n_pre])
 *   grad_w[s]   = x[i] * g[idx[s]] for every synapse s of row i    (w != NULL; [nnz or n_pre*k])
 *   grad_w[0]   = sum_i x[i] * sum_k g[idx[i,k]]                    (w == NULL; one scalar)
 * Rows are fixed-num (indptr == NULL) or CSR as in bs_event_scatter_f32.  Out-of-range targets
 * contribute nothing.  Sums are fp32 in an unspecified order. */
BS_API int bs_event_matvec_vjp_f32(const void* spk, int32_t spk_dtype, int32_t n_pre,
                                   const int32_t* indptr, const int32_t* indices, int32_t k,
                                   const float* w, float w_homo, int32_t n_post,
                                   const float* grad_out, float* grad_spk, float* grad_w,
                                   bs_stream_t stream);
/* The same for `batch` rows (spk [batch, n_pre], grad_out [batch, n_post], grad_spk [batch,
 * n_pre]) in one launch, the reverse mode of bs_event_matvec_batch_f32 (the batched module's
 * gradient, brainstate/nn/_event_fixedprob.py:202-209 under init_all_states(batch_size)):
 * grad_spk row b as bs_event_matvec_vjp_f32 gives it for row b; per-synapse grad_w[s] =
 * sum_b x[b, i] * g[b, idx[s]] with the products added in row order (the per-row gradients
 * added one after another); a homogeneous grad_w[0] sums over rows and synapses. */
BS_API int bs_event_matvec_vjp_batch_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                         int32_t n_pre, const int32_t* indptr,
                                         const int32_t* indices, int32_t k, const float* w,
                                         float w_homo, int32_t n_post, const float* grad_out,
                                         float* grad_spk, float* grad_w, bs_stream_t stream);

/* ---------------------------------------------------------------- N2a, destination-bucketed
 * Same operator as bs_event_scatter_f32 / bs_event_matvec_f32 (replaces `EventArray(spk) @
 * FixedPostNumConn` / `@ CSR`, brainstate/nn/_event_fixedprob.py:176-181,192,202-205,249-252)
 * with no global atomics and no fp32 atomics, on a layout built once per connectivity:
 *   nb = bs_bucket_plan(n_post, &P): posts are cut into nb buckets of P consecutive posts
 *        (bucket b holds [b*P, min((b+1)*P, n_post)), P <= 12288, nb <= 1024);
 *   bs_bucket_build: seg[n_pre][nb+1] (int32), lidx[nnz] (uint16), lw[nnz] (fp32 or NULL)
 *        and, with per-synapse weights, the fixed-point exponent *qexp (device int32;
 *        `workspace` = 4 * (n_post + 1) device bytes of scratch).  Row i's synapses stay
 *        inside [indptr[i], indptr[i+1]) (fixed-num: [i*k, i*k+k)), sorted by bucket with the
 *        original order kept inside a bucket; bucket b's synapses of row i are
 *        [seg[i][b], seg[i][b+1]) with lidx = target - b*P; valid synapses end at seg[i][nb]
 *        (out-of-range targets follow and are never read).  S = *qexp = min(30 - e_w - e_d,
 *        100) with max|w| < 2^e_w over the valid synapses (e_w from the exponent field, -126
 *        for 0 or a subnormal) and the largest number of valid synapses onto one post
 *        D <= 2^e_d: the persistent runner's rule (bs_net_prepare), so a projection gives the
 *        same sums here and inside the runner; every output's sum of rounded weights stays
 *        below 2^30 in magnitude (-1000 if a weight is not finite or S < -100).
 * bs_event_bucket_f32: out[j] = (accumulate ? out[j] : 0) + v_j, where v_j is
 *   - per-synapse weights, finite: each weight of an event onto j rounded to a multiple of
 *     2^-S (round to nearest even), the rounded weights summed exactly (32-bit integers),
 *     the sum rounded once to fp32 and scaled by 2^-S: deterministic, whatever the order of
 *     the device's atomics;
 *   - homogeneous weight (lw == NULL): w_homo added once per event onto j, in one chain
 *     starting from out[j] (or 0): bit-identical to a sequential scatter;
 *   - a non-finite per-synapse weight: fp32 sums in an unspecified order.
 * The step is one kernel over nb x R row groups plus a reduce of the partials.  mode:
 *   0  R follows the spikes on the device (about 128 active rows per group, estimated from
 *      the leading 16,384 rows; at R = 1 the reduce has nothing to do);
 *   1  one launch of nb x min(8, 256 / nb) workgroups that write out themselves, no estimate
 *      (R = 1 whatever the density: right for sparse spikes, slow for dense ones);
 *   2  R = its maximum (row_groups), fixed on the host: no estimate on the critical path
 *      (right for dense spikes); a layout whose maximum is 1 (n_pre <= 64, or more than
 *      128 buckets) runs as mode 0.
 * The sums are the same bits in every mode.  est_out (NULL, or an int32 the device can write,
 * e.g. in pinned host memory) receives the call's estimate of R (mode 0: from the leading
 * rows; mode 1: ceil(active rows / 128) from the exact count; mode 2: from row group 0), so that a caller can pick the next call's mode from it without a
 * synchronisation (a stale estimate costs time, never correctness).
 * `workspace`: bs_event_bucket_workspace_size bytes (mode 1: 256 bytes are enough), 8-byte
 * aligned, no initialisation needed. */
BS_API int bs_bucket_plan(int32_t n_post, int32_t* P_out);
BS_API int bs_bucket_build(int32_t n_pre, const int32_t* indptr, const int32_t* indices, int32_t k,
                           const float* w, int32_t n_post, int32_t nb, int32_t P, int32_t* seg,
                           uint16_t* lidx, float* lw, int32_t* qexp, void* workspace,
                           bs_stream_t stream);
BS_API size_t bs_event_bucket_workspace_size(int32_t n_pre, int32_t n_post, int32_t nb);
BS_API int bs_event_bucket_f32(const void* spk, int32_t spk_dtype, int32_t n_pre, int32_t n_post,
                               int32_t nb, int32_t P, const int32_t* seg, const uint16_t* lidx,
                               const float* lw, const int32_t* qexp, float w_homo, float* out,
                               int32_t accumulate, void* workspace, size_t workspace_bytes,
                               int32_t mode, int32_t* est_out, bs_stream_t stream);

/* ---------------------------------------------------------------- N2b event gather
 * Same operator as N2a, post-major and deterministic (no atomics).  Spikes come as a
 * bitmap (bs_spike_pack: bit i%32 of word i/32 set <=> spk[i] != 0).  Layout SELL-64x4:
 * posts are grouped in slices of 64; slice s holds ncol(s) columns (a multiple of 4) of
 * incoming synapses, column c of post lane (= post - 64*s) at
 * sell_pre[slice_ptr[s] + (c/4)*256 + lane*4 + c%4] (each lane's 4 consecutive columns are
 * one 16-byte word), columns in ascending (pre, k) order, padded with -1; slice_ptr[s] is a
 * multiple of 256 and sell_pre / sell_w are 16-byte aligned.  out[j] = 0.0f + the weights
 * of active synapses in that order, i.e. bit-identical to a sequential pre-major scatter.
 * sell_w == NULL -> homogeneous w_homo.  n_slices = ceil(n_post / 64). */
BS_API int bs_spike_pack(const void* spk, int32_t spk_dtype, int32_t n, uint32_t* bits,
                         bs_stream_t stream);
BS_API int bs_event_gather_f32(const uint32_t* spk_bits, int32_t n_pre,
                               const int64_t* slice_ptr, const int32_t* sell_pre,
                               const float* sell_w, float w_homo, int32_t n_post, float* out,
                               bs_stream_t stream);

/* ---------------------------------------------------------------- N2c event x dense
 * Replaces `EventArray(spk) @ W` / `spk @ W` of EventLinear
 * (brainstate/nn/_event_linear.py:99-102).  spk [batch, n_in], W [n_in, n_out] row-major,
 * out [batch, n_out].  float_as_event != 0: out[b] = sum of rows W[i] with spk[b,i] != 0;
 * otherwise out[b] = sum_i spk[b,i] * W[i].
 * Order of the fp32 additions (fixed by the shape alone): the inputs are split into
 * S = bs_event_dense_chunks(batch, n_in, n_out, &L) chunks of L consecutive rows (L a multiple
 * of 64; the last chunk may be shorter); P_c = the chunk's terms added in ascending i starting
 * from 0; out = ((P_0 + P_1) + P_2) + ... + P_{S-1}.  S = 1 is the plain ascending sum.
 * `workspace` holds bs_event_dense_workspace_size(batch, n_in, n_out) bytes (0 when S = 1,
 * then it may be NULL).  Its first bs_event_dense_ticket_bytes(batch, n_in, n_out) bytes are
 * ticket counters: they must be zero on entry and the call leaves them zero; the rest holds
 * partial sums and needs no initialisation.  A workspace zero-filled once therefore serves any
 * sequence of calls whose ticket bytes do not grow; before a call whose ticket bytes exceed
 * the previous call's, zero the difference.  Calls that share a workspace must be ordered on
 * one stream. */
BS_API int bs_event_dense_chunks(int32_t batch, int32_t n_in, int32_t n_out, int32_t* chunk_rows);
BS_API size_t bs_event_dense_workspace_size(int32_t batch, int32_t n_in, int32_t n_out);
BS_API size_t bs_event_dense_ticket_bytes(int32_t batch, int32_t n_in, int32_t n_out);
BS_API int bs_event_dense_f32(const void* spk, int32_t spk_dtype, int32_t batch, int32_t n_in,
                       const float* W, int32_t n_out, int32_t float_as_event, float* out,
                       void* workspace, size_t workspace_bytes, bs_stream_t stream);

/* Packed form of the same product for byte / event spikes (float_as_event semantics: any
 * nonzero spike is an event), for a W that is reused across calls.  Exact in fixed point:
 * column j is scaled by 2^S_j, S_j = D - e_j, D = 8 L - 2, where max_i |W[i,j]| = f * 2^e_j with
 * f in [0.5, 1) and L = bs_event_dense_digits(n_in) (4, 5 or 6: the smallest with
 * D >= 24 + ceil(log2 n_in); 0 when n_in > 65536, which the packed form does not take).
 * q[i,j] = rint(W[i,j] * 2^S_j) (ties to even); out[b,j] = ldexp((float) sum of q[i,j] over
 * the inputs with spk[b,i] != 0, -S_j): one rounding of an exact integer sum, so the result
 * does not depend on any order, and the weight rounding moves a sum by at most
 * 2^-24 * max_i |W[i,j]|.  A column of zeros gives +0.
 * bs_event_dense_pack(W, ...) fills `packed` (bs_event_dense_packed_bytes(n_in, n_out) bytes,
 * 256-byte aligned): a header whose first uint32 is the status (1 when a weight is inf or
 * NaN: then every output of bs_event_dense_packed_f32 is NaN; use bs_event_dense_f32), the
 * column maxima and the digits (layout in csrc/event_dense_packed.hip).  It must be redone
 * after W changes.  bs_event_dense_packed_f32 reads it (n_in, n_out as packed), spk u8 or
 * f32 [batch, n_in], and writes out [batch, n_out]; no workspace.  Replaces the same call
 * as bs_event_dense_f32 (brainstate/nn/_event_linear.py:99-100) when one W serves many calls
 * (recurrent loops over time, inference). */
BS_API int32_t bs_event_dense_digits(int32_t n_in);
BS_API int64_t bs_event_dense_packed_bytes(int32_t n_in, int32_t n_out);
BS_API int bs_event_dense_pack(const float* W, int32_t n_in, int32_t n_out, void* packed,
                               int64_t packed_bytes, bs_stream_t stream);
BS_API int bs_event_dense_packed_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                     int32_t n_in, const void* packed, int32_t n_out, float* out,
                                     bs_stream_t stream);

/* Reverse mode of EventLinear's heterogeneous product (the VJP the reference checks at
 * brainstate/nn/_event_linear_test.py:51-89; its "true gradient" is that of x @ W with the
 * spike values x, 0/1 for byte spikes, in both float_as_event modes):
 *   grad_spk[b,i] = sum_j grad_out[b,j] * W[i,j]     (nullable, [batch, n_in])
 *   grad_W[i,j]   = sum_b x[b,i] * grad_out[b,j]     (nullable, [n_in, n_out]; every element
 *                                                     written, rows no spike selects get 0)
 * fp32 with fused multiply-adds; grad_spk sums are reduced across a wave, grad_W sums run
 * in ascending b. */
BS_API int bs_event_dense_vjp_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                  int32_t n_in, const float* W, int32_t n_out,
                                  const float* grad_out, float* grad_spk, float* grad_W,
                                  bs_stream_t stream);

/* ---------------------------------------------------------------- N3 fused updates
 * LIF / LIFRef membrane with Expon synapses and COBA output -- the per-step elementwise
 * work of brainpy.state LIFRef + Expon + COBA + AlignPostProj as driven by
 * brainstate/nn/_exp_euler.py:226-249 (used e.g. by examples/105_COBA_HH_2007_braincell.py:62-82).
 *   g_e = g_e*decay_e + in_e;  g_i = g_i*decay_i + in_i
 *   I = I_ext + g_e*(E_e - V) + g_i*(E_i - V)
 *   V' = V + (dt*exprel(dt*J))*f,  f = ((V_rest - V) + R*I)*inv_tau,  J = (-1 - R*(g_e+g_i))*inv_tau
 *   refractory (ref > 0): V held, ref -= 1;  else spike = V' >= V_th -> V' = V_reset,
 *   ref = ref_steps.
 * inv_tau = fp32(1/tau): the reference's `/ tau` by a constant, as XLA executes it. */
typedef struct {
  float V_rest, V_th, V_reset, inv_tau, R, I_ext, E_e, E_i, dt, decay_e, decay_i;
  int32_t ref_steps;
  /* cuba != 0: current-based output (brainpy.state CUBA, used by
   * examples/400_CUBA_2005_bpu.py:42-58): I = I_ext + g_e*scale_e + g_i*scale_i (one fused
   * multiply-add each), J = -inv_tau; E_e / E_i are then unused.  cuba == 0: COBA as above. */
  int32_t cuba;
  float scale_e, scale_i;
  /* soft_reset != 0 (brainpy.state LIF spk_reset='soft', used by
   * docs/tutorials/brain_dynamics/04_building_an_snn.ipynb cells 5, 11): a spike subtracts
   * (V_th - V_reset) from V' instead of setting V' = V_reset. */
  int32_t soft_reset;
  /* deferred_reset != 0: the reset of a spike is applied at the start of the neuron's next
   * step, as brainpy.state's neurons do (`last_V = V - (V_th - V_reset) * last_spk` before the
   * update; the reference-held neuron of examples/203_braintrace_for_snns.py:173-176): a
   * spiking neuron keeps V' >= V_th in V until then.  Spike rasters and every other state
   * are those of deferred_reset == 0.  bs_coba_lif_step then reads the previous step's
   * spikes from spk_out before it overwrites them; the runners take them from net->spk. */
  int32_t deferred_reset;
} bs_lif_params;

BS_API int bs_coba_lif_step(int32_t n, float* V, float* ge, float* gi, int32_t* ref,
                     const float* in_e, const float* in_i, const bs_lif_params* p,
                     uint8_t* spk_out, bs_stream_t stream);
/* Per-neuron LIF parameters: each non-NULL array [n] replaces the scalar of bs_lif_params
 * for its neuron (a population built with array-valued V_rest, V_th, V_reset, tau, R or
 * tau_ref; inv_tau = fp32(1 / tau), ref_steps = the refractory steps of that neuron's tau_ref). */
typedef struct {
  const float* V_rest; const float* V_th; const float* V_reset; const float* inv_tau;
  const float* R; const int32_t* ref_steps;
} bs_lif_arrays;

/* The same step with a per-neuron external input: I_ext [n] (NULL: p->I_ext for every
 * neuron) in place of p->I_ext, as when the reference's neuron is called with an input array
 * (brainpy.state LIFRef.update(x), x of the population's shape). */
BS_API int bs_coba_lif_step_in(int32_t n, float* V, float* ge, float* gi, int32_t* ref,
                               const float* in_e, const float* in_i, const float* I_ext,
                               const bs_lif_params* p, uint8_t* spk_out, bs_stream_t stream);
/* ... and with per-neuron parameters (arr NULL, or any of its arrays NULL: the scalars). */
BS_API int bs_coba_lif_step_arr(int32_t n, float* V, float* ge, float* gi, int32_t* ref,
                                const float* in_e, const float* in_i, const float* I_ext,
                                const bs_lif_arrays* arr, const bs_lif_params* p,
                                uint8_t* spk_out, bs_stream_t stream);

/* One recurrent step of a packed EventLinear driving COBA-LIF neurons, in one launch:
 * cur = the bs_event_dense_packed_f32 product of spk [batch, n_in] with `packed`, then the
 * bs_coba_lif_step update of the [batch, n_out] state (V, ge, gi, ref) with in_e = cur,
 * in_i = 0 (inh = 0) or in_e = 0, in_i = cur (inh != 0).  The bits equal those two calls in
 * sequence.  cur_out (nullable) receives cur; spk_out (nullable) the spikes as 0/1 bytes.
 * No output (spk_out, cur_out, V, ge, gi, ref) may overlap the spike input -- a recurrent
 * caller double-buffers the spikes; an overlap is rejected with BS_ERR_INVALID.
 * Replaces EventLinear (brainstate/nn/_event_linear.py:99-100) followed by the Expon + COBA +
 * LIFRef update it feeds (brainstate/nn/_exp_euler.py:226-249). */
BS_API int bs_event_dense_packed_lif_step(const void* spk, int32_t spk_dtype, int32_t batch,
                                          int32_t n_in, const void* packed, int32_t n_out,
                                          int32_t inh, float* V, float* ge, float* gi,
                                          int32_t* ref, const bs_lif_params* p, float* cur_out,
                                          uint8_t* spk_out, bs_stream_t stream);

/* Hodgkin-Huxley with Expon synapses and COBA output (examples/100_hh_neuron_model.py:25-93):
 * rates from the old V; V, m, h, n each by exp-Euler; spike = (V < V_th) & (V' >= V_th). */
typedef struct {
  float ENa, gNa, EK, gK, EL, gL, inv_C, V_th, I_ext, E_e, E_i, dt, decay_e, decay_i;
} bs_hh_params;   /* inv_C = fp32(1/C) */

/* One exponential-Euler step of a general drift, elementwise over n values:
 *   out = x + (dt * exprel(dt * jac)) * drift     (one fused multiply-add; exprel as above)
 * drift = f(x, ...) and jac = the vector-Jacobian product of f with ones (the diagonal of
 * df/dx for an elementwise f), both computed by the caller.  Replaces the arithmetic of
 * brainstate.nn.exp_euler_step (brainstate/nn/_exp_euler.py:206-249).  out may alias x.
 * The f64 form uses exprel(z) = expm1(z) / z (series below |z| = 1e-3). */
BS_API int bs_exp_euler_f32(int64_t n, const float* x, const float* drift, const float* jac,
                            float dt, float* out, bs_stream_t stream);
BS_API int bs_exp_euler_f64(int64_t n, const double* x, const double* drift, const double* jac,
                            double dt, double* out, bs_stream_t stream);

/* Gates at steady state for V (examples/100_hh_neuron_model.py:66-70). */
BS_API int bs_hh_init(int32_t n, const float* V, float* m, float* h, float* ng, bs_stream_t stream);
BS_API int bs_coba_hh_step(int32_t n, float* V, float* m, float* h, float* ng, float* ge, float* gi,
                    const float* in_e, const float* in_i, const bs_hh_params* p,
                    uint8_t* spk_out, bs_stream_t stream);
/* Per-neuron HH parameters: each non-NULL array [n] replaces the scalar of bs_hh_params for
 * its neuron (inv_C = fp32(1 / C)). */
typedef struct {
  const float* ENa; const float* gNa; const float* EK; const float* gK; const float* EL;
  const float* gL; const float* inv_C; const float* V_th;
} bs_hh_arrays;

/* The same step with a per-neuron external input I_ext [n] (NULL: p->I_ext), as for an input
 * array passed to the HH neuron (examples/100_hh_neuron_model.py:72-93 with x of shape [n]). */
BS_API int bs_coba_hh_step_in(int32_t n, float* V, float* m, float* h, float* ng, float* ge,
                              float* gi, const float* in_e, const float* in_i,
                              const float* I_ext, const bs_hh_params* p, uint8_t* spk_out,
                              bs_stream_t stream);
/* ... and with per-neuron parameters (arr NULL, or any of its arrays NULL: the scalars). */
BS_API int bs_coba_hh_step_arr(int32_t n, float* V, float* m, float* h, float* ng, float* ge,
                               float* gi, const float* in_e, const float* in_i,
                               const float* I_ext, const bs_hh_arrays* arr,
                               const bs_hh_params* p, uint8_t* spk_out, bs_stream_t stream);

/* ---------------------------------------------------------------- whole-loop runners
 * Replace `brainstate.transform.for_loop(net.update, times)` over an E/I network
 * (brainstate/transform/_loop_collect_return.py:487-572 -> jax.lax.scan at :268) for the
 * two projections E: neurons [0, n_exc) -> all n, I: [n_exc, n) -> all n, each
 * fixed-num (brainstate/nn/_event_fixedprob.py:102-205), in the per-step order of
 * examples/105_COBA_HH_2007_braincell.py:76-82 (previous step's spikes -> event mat-vecs ->
 * neuron update).  One persistent launch runs `steps` network steps with no grid barrier:
 * events travel through per-(source, destination) workgroup inboxes sized from the
 * connectivity, so they cannot overflow.
 * Protocol: bs_net_prepare() once per (net, workspace) -- it sizes the inboxes and clears
 * the pending events -- then runs with consecutive absolute step indices t0 = 0, s1,
 * s1+s2, ...  State arrays are read at the start and written at the end of each run;
 * spk receives the last step's spikes.  w_e/w_i == NULL -> homogeneous w_*_homo.
 * counts_out[t] / hash_out[t] (nullable): number of spikes and the order-free digest
 * sum_i mix32(i) mod 2^32 of step t; raster_out [steps, n] uint8 (nullable). */
typedef struct {
  int32_t n, n_exc, k_e, k_i;
  const int32_t* idx_e; const float* w_e; float w_e_homo;   /* [n_exc, k_e] */
  const int32_t* idx_i; const float* w_i; float w_i_homo;   /* [n - n_exc, k_i] */
  uint8_t* spk;                                             /* [n] last step's spikes */
  int32_t blocks_per_cu;                                    /* 0 = library default */
  int32_t delay_steps;   /* synaptic delay D in [0, 1023]: step t's inputs come from the spikes
                            of step t-1-D, as `N.prefetch_delay('spike', D*dt)` gives
                            (brainstate/nn/_dynamics.py:222-262, _delay.py:762-790); no spikes
                            before the first step; workspace grows as 2(D+1) inbox slots */
  const float* I_ext;    /* [n] per-neuron constant external input, in place of the neuron
                            parameters' I_ext (NULL: the parameters' I_ext for every neuron),
                            as a script calling N(x) with an input array x of shape [n] */
} bs_net;

typedef struct { float* V; float* ge; float* gi; int32_t* ref; } bs_lif_state;
typedef struct { float* V; float* m; float* h; float* n; float* ge; float* gi; } bs_hh_state;

/* Workspace bytes for this net on the current device (0 on error; about
 * 2(D+1) x synapses x (8 B heterogeneous | 4 B homogeneous)). */
BS_API size_t bs_net_workspace_size(const bs_net* net);
BS_API int bs_net_prepare(const bs_net* net, void* workspace, bs_stream_t stream);
BS_API int bs_coba_lif_run(const bs_net* net, const bs_lif_state* st, const bs_lif_params* p,
                           int64_t t0, int32_t steps, int32_t* counts_out, uint32_t* hash_out,
                           uint8_t* raster_out, void* workspace, bs_stream_t stream);
BS_API int bs_coba_hh_run(const bs_net* net, const bs_hh_state* st, const bs_hh_params* p,
                          int64_t t0, int32_t steps, int32_t* counts_out, uint32_t* hash_out,
                          uint8_t* raster_out, void* workspace, bs_stream_t stream);
/* The same runs with an external input per step: I_steps [steps] (device, fp32) is step
 * t0 + k's input in place of p->I_ext, as a loop over xs passes each step its own x
 * (`for_loop(f, xs)`, brainstate/transform/_loop_collect_return.py:487-572, whose scan body
 * calls N(x_t)); one launch however the input changes.  Not combined with net->I_ext. */
BS_API int bs_coba_lif_run_inputs(const bs_net* net, const bs_lif_state* st,
                                  const bs_lif_params* p, const float* I_steps, int64_t t0,
                                  int32_t steps, int32_t* counts_out, uint32_t* hash_out,
                                  uint8_t* raster_out, void* workspace, bs_stream_t stream);
BS_API int bs_coba_hh_run_inputs(const bs_net* net, const bs_hh_state* st,
                                 const bs_hh_params* p, const float* I_steps, int64_t t0,
                                 int32_t steps, int32_t* counts_out, uint32_t* hash_out,
                                 uint8_t* raster_out, void* workspace, bs_stream_t stream);

/* Pending spikes for a run that starts at step t0 >= 1 (synaptic delay 0): spk [n] (nonzero
 * = spike) are taken as the spikes of step t0 - 1, so step t0's inputs come from them, as
 * when the loop was advanced step by step elsewhere (brainstate.transform.for_loop handing
 * over after its first steps).  Call after bs_net_prepare, before the run from t0. */
BS_API int bs_net_seed_spikes(const bs_net* net, const uint8_t* spk, int64_t t0,
                              void* workspace, bs_stream_t stream);

/* Workgroups the runners use for this net on the current device (-1 on error). */
BS_API int bs_net_grid_blocks(const bs_net* net);
/* Synchronises `stream`; returns 0 if every wait of the runs so far completed, -1 if one
 * hit its spin limit (results invalid), -2 if bs_net_prepare found a per-synapse weight that
 * is not finite (results invalid), or a positive status on a call failure. */
BS_API int bs_net_error(const void* workspace, bs_stream_t stream);

/* ---------------------------------------------------------------- connectivity on the device
 * FixedNumConn's index draws (brainstate/nn/_event_fixedprob.py:142-196) without the host.
 *
 * bs_conn_fixed_num: indices [n_pre * k] equal, bit for bit, to
 * numpy.random.RandomState(seed).randint(0, n_post, (n_pre, k)) (:163-168); when `selected`
 * is given, selected[i] = (rng.random(n_pre) < afferent_ratio)[i] drawn next from the same
 * stream (:186).  With k == 0 `selected` is the first n_pre draws of random().  Synchronises
 * `stream` once (the generator reports how far the stream was consumed).  Workspace:
 * bs_conn_fixed_num_workspace_size (about 4 B per draw). */
BS_API size_t bs_conn_fixed_num_workspace_size(int32_t n_pre, int32_t k, int32_t n_post,
                                               int32_t with_selection);
BS_API int bs_conn_fixed_num(uint32_t seed, int32_t n_pre, int32_t k, int32_t n_post,
                             int32_t* indices, double afferent_ratio, uint8_t* selected,
                             void* workspace, size_t workspace_bytes, bs_stream_t stream);
/* CSR of the selected rows (:185-196): indptr[i + 1] = k * (selected rows <= i); when `out` is
 * given, the selected rows of indices [n_pre, k] are copied to out[indptr[i] ..] in order. */
BS_API int bs_csr_from_selected(const int32_t* indices, int32_t n_pre, int32_t k,
                                const uint8_t* selected, int32_t* indptr, int32_t* out,
                                bs_stream_t stream);
/* allow_multi_conn=False (init_indices_without_replace, :39-62): k <= 2048 distinct targets
 * per row, uniform over [0, n_post), from Philox4x32-10 keyed by `seed`.  The reference draws
 * these with its JAX generator, whose stream is not reproduced. */
BS_API int bs_conn_fixed_num_unique(uint64_t seed, int32_t n_pre, int32_t k, int32_t n_post,
                                    int32_t* indices, bs_stream_t stream);

/* ---------------------------------------------------------------- ring-buffer delay
 * Device side of brainstate's Delay / StateWithDelay (brainstate/nn/_delay.py:399-1079): a
 * history of `length` slots, slot-major, each `slot_elems` elements (a slot holds one value of
 * the delayed state, batch included).  The ring index arithmetic -- write slot
 * write_ptr // update_every_step, newest slot cur = (write_ptr - 1) // update_every_step,
 * read slot (cur - step) mod length (:772-790, :909-928) -- is the caller's; these copy.
 *
 * bs_delay_write: copy `slot_bytes` from src into slot `slot` (replaces
 * `history.at[idx].set(value)`, _delay.py:917-921). */
BS_API int bs_delay_write(void* hist, int32_t length, int64_t slot_bytes, int32_t slot,
                          const void* src, bs_stream_t stream);
/* bs_delay_gather: out[j] = hist[((cur - s_j) mod length) * slot_elems + c_j] for elements of
 * elem_bytes in {1, 2, 4, 8}, with s_j = steps ? steps[j] : step and c_j = cols ? cols[j] : j
 * (cols, when given, must lie in [0, slot_elems)).  Replaces `retrieve_at_step(delay_step,
 * *indices)` (:762-790): a scalar step copies one slot; step / index arrays are the fancy
 * indexing of vector delays, broadcast and flattened to (steps, cols) by the caller. */
BS_API int bs_delay_gather(const void* hist, int32_t length, int64_t slot_elems,
                           int32_t elem_bytes, int32_t cur, int32_t step, const int32_t* steps,
                           const int64_t* cols, int64_t n_out, void* out, bs_stream_t stream);
/* bs_delay_taps_f32: out[j] = sum_{q < taps} weights[q] * hist[slots[q] * slot_elems + c_j],
 * products rounded then added left to right; slots / weights are host arrays of at most 4.
 * Replaces the continuous-time reads of `retrieve_at_time` (:798-907) with the interpolation
 * methods of :163-338 (linear: 2 taps; polynomial2: 3; cubic, hermite, polynomial3: 4). */
BS_API int bs_delay_taps_f32(const float* hist, int32_t length, int64_t slot_elems, int32_t taps,
                             const int32_t* slots, const float* weights, const int64_t* cols,
                             int64_t n_out, float* out, bs_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BRAINSTATE_AMD_H_ */

// Whole-loop runners for E/I networks: one persistent (cooperative) launch runs T steps.
//
// Why persistent: one step of the 1M-neuron COBA net moves ~34 MB, ~4 us at 8 TB/s, the
// same order as a kernel launch, so a per-step chain of launches is launch-bound.  Each
// workgroup owns a fixed power-of-two slice of neurons for the whole run and keeps their
// state in registers.
//
// Why no global atomics: scattered fp32 atomics on MI355X sustain ~20 G/s chip-wide
// (scattered plain stores ~80 G/s), so atomically scattering ~2e5 synaptic events per
// step would cost > 9 us by itself.  Instead events travel through per-(source, destination)
// inboxes, which connectivity makes boundable: the number of synapses from the neurons of
// workgroup s onto those of workgroup d is fixed, so each inbox is sized for the case in
// which every neuron of s spikes and can never overflow (the whole structure is
// 2 x synapses x 8 B, e.g. 1.6 GB for 1e8 synapses; HBM is 288 GB).
//
// Per step t, workgroup d:
//   A. waits until every workgroup s has published its step t-1-D count word for d (tagged
//      with the step; D = synaptic delay in steps, 0 by default) and adds the entries of
//      that inbox into two 32-bit LDS words per neuron (E, I) with integer LDS atomics --
//      point-to-point dependencies, no grid barrier;
//   B. runs the fused Expon + COBA + neuron update from those inputs;
//   C. compacts its spikes into an LDS list (one ballot per neuron slot, one LDS prefix);
//   D. expands its spikes into (local target | inh flag, weight) entries, written with
//      device-scope stores at slots taken from per-destination LDS cursors; each wave waits
//      for its own stores to complete and publishes the tagged count words of the
//      destinations it wrote (all waves' stores first when an entry overflowed the slots).
//
// Input sums are integers, so they do not depend on the order in which entries arrive:
//   * one weight per projection (homogeneous): the words count events; the input is w added
//     c times in one fp32 chain (c = count), which is what a sequential scatter of one
//     repeated value gives in any order;
//   * per-synapse weights: each weight is rounded to a multiple of 2^-S (S per projection,
//     fixed at prepare from the largest |w| and the largest in-degree so that no sum can
//     leave int32), the words hold the two's-complement int32 sums, and the input is the sum
//     converted to fp32 (one rounding) times 2^-S.
// Cross-workgroup data is only touched with device-scope loads/stores (emitted with the
// device-coherence bit), so no L2 writeback/invalidate is ever needed (each costs ~5 us).
// Deadlock freedom: every workgroup publishes step t's counts unconditionally after
// consuming step t-1-D's, and all workgroups are co-resident (cooperative launch); a spin
// limit turns a would-be hang into an error flag instead.
// Ring of R = 2(D+1) inbox / count-word slots, step u in slot u mod R: a workgroup at step t
// has seen every workgroup's step t-1-D publication, so none is more than D+1 steps behind
// it; the slowest one, at step t-D, still reads step t-2D-1's entries, and R slots keep those
// (and everything newer) from being overwritten.  With D = 0 this is double buffering; with
// D > 0 the entries a step consumes were published D steps earlier, so its waits are short.
#include "neuron_dev.h"

namespace {

constexpr int kBlock = 1024;
constexpr int kWaves = kBlock / BS_WAVE;
constexpr int kMaxBlocks = 256;
constexpr int kMaxNpt = 8;
constexpr uint32_t kInhFlag = 0x80000000u;
constexpr uint64_t kSpinLimit = 1ull << 24;
constexpr int kRunSteps = 16384;          // steps per cooperative launch (partials buffer)
constexpr int kMaxDelay = 1023;           // synaptic delay in steps (ring of 2(D+1) slots)
#ifndef BS_POLL_SLEEP
#define BS_POLL_SLEEP 1  // s_sleep units (64 clocks) between polls of a count word
#endif
#define BS_AGENT __HIP_MEMORY_SCOPE_AGENT


// ---- workspace layout (all offsets in bytes, 256-aligned) ----
struct NetLayout {
  int32_t nb;          // workgroups
  int32_t npt;         // neurons per thread
  int32_t shift;       // log2(neurons per workgroup)
  uint32_t entry;      // bytes per entry (8 het, 4 homogeneous)
  int32_t delay;       // synaptic delay D in steps
  int32_t ring;        // inbox / count-word slots R = 2(D+1)
  uint64_t total;      // inbox entries per slot (>= valid synapses)
  uint64_t off_cnt;    // uint64 [R][nb dst][nb src]   tagged counts
  uint64_t off_cap;    // uint32 [nb src][nb dst]      capacities
  uint64_t off_ofs;    // uint64 [nb dst][nb src] + 1  inbox entry offsets (dst-major)
  uint64_t off_part;   // uint32 [2][kRunSteps][nb]  per-workgroup spike counts / hashes
  uint64_t off_deg;    // uint32 [2][n]  in-degree per kind (prepare, per-synapse weights)
  uint64_t off_vprev;  // fp32 [n]  V before a run's last step (deferred reset)
  uint64_t off_inbox;  // entries [R][total]
  uint64_t bytes;
};

struct WsHeader {
  uint32_t error;      // 1: a wait hit the spin limit; 2: a per-synapse weight is not finite
  int32_t qexp[2];     // fixed-point exponents S_e, S_i of per-synapse weights (prepare)
  uint32_t wbits[2];   // bit patterns of max |w| per kind (prepare)
  uint32_t pad[59];
};
static_assert(sizeof(WsHeader) == 256, "workspace header is 256 bytes");

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__device__ __forceinline__ uint64_t ld_dev64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, BS_AGENT);
}
__device__ __forceinline__ void st_dev64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, BS_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, BS_AGENT);
}
__device__ __forceinline__ void st_dev32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, BS_AGENT);
}

struct NetArgs {
  int32_t n, n_exc, k_e, k_i;
  const int32_t* idx_e;
  const float* w_e;
  float w_e_homo;
  const int32_t* idx_i;
  const float* w_i;
  float w_i_homo;
  uint8_t* spk;
  int64_t t0;
  int32_t steps;
  int32_t slot_rd;   // ring slot of step t0-1-D (the entries the first step consumes)
  int32_t slot_wr;   // ring slot of step t0
  uint32_t* counts;  // per-workgroup spike counts [steps][nb] (workspace), or NULL
  uint32_t* hash;    // per-workgroup spike hashes [steps][nb] (workspace), or NULL
  uint8_t* raster;
  const float* iext;  // per-neuron external input [n], or NULL (the parameters' I_ext)
  const float* isched;  // external input of each step of the launch [steps], or NULL
  char* ws;
  NetLayout L;
};

// One float of a read-only input array, loaded into a VGPR (a vector load: a scalar load
// would share the LDS accesses' wait counter, and the next LDS wait would wait for it too).
__device__ __forceinline__ float ld_input(const float* p) {
  return __uint_as_float(
      __hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}

// The parameters with a neuron's own external input.
template <class P>
__device__ __forceinline__ P with_input(P p, float x) {
  p.I_ext = x;
  return p;
}

// ---- neuron models: register-resident state, one fused update per neuron-step ----

template <bool kCuba, bool kSoft>
struct LifModel {
  using Params = bs_lif_params;
  using State = bs_lif_state;
  struct Regs {
    float V, ge, gi;
    int32_t ref;
  };
  __device__ static Regs load(const State& s, int64_t j) {
    return Regs{s.V[j], s.ge[j], s.gi[j], s.ref[j]};
  }
  __device__ static void store(const State& s, int64_t j, const Regs& r) {
    s.V[j] = r.V;
    s.ge[j] = r.ge;
    s.gi[j] = r.gi;
    s.ref[j] = r.ref;
  }
  static constexpr bool kPrepare = false;  // every operation of the step needs the input
  // parameters and row pointers held in VGPRs (see k_run)
  static constexpr bool kParamVgprs = true;
  // count words published by the loop over write-out slots (see k_run)
  static constexpr bool kPubByLane = false;
  __device__ static void prepare(const Params&, Regs&) {}
  __device__ static bool update(const Params& p, Regs& r, float in_e, float in_i) {
    return bs_lif_update<kCuba, kSoft>(p, r.V, r.ge, r.gi, r.ref, in_e, in_i);
  }
  // Whether the neuron may spike this step: a zero-input forward-Euler estimate of the next
  // V within 7 % of (V_th - V_reset) of threshold.  Only steers the row prefetch; the
  // estimate never decides a spike.  Measured on the 1M-neuron COBA-LIF net (us per step): margin 0.02 7.45,
  // 0.05 7.24, 0.07 7.235, 0.10 7.25, 0.15 7.33, 0.20 7.51; V alone against a 0.15 / 0.25
  // margin 7.96 / 8.13 (too many rows); extrapolating V by the step's own change 7.76-8.03
  // (misses the neurons the next input pushes over).
  __device__ static bool near(const Params& p, const Regs& r) {
    const float I = kCuba ? p.I_ext + r.ge * p.decay_e * p.scale_e + r.gi * p.decay_i * p.scale_i
                          : p.I_ext + r.ge * p.decay_e * (p.E_e - r.V) +
                                r.gi * p.decay_i * (p.E_i - r.V);
    const float vp = r.V + p.dt * p.inv_tau * ((p.V_rest - r.V) + p.R * I);
    return r.ref <= 0 && vp >= p.V_th - 0.07f * (p.V_th - p.V_reset);
  }
};

struct HhModel {
  using Params = bs_hh_params;
  using State = bs_hh_state;
  struct Regs {
    float V, m, h, n, ge, gi;
    bs_hh_pre pre;  // input-independent part of the coming step
  };
  __device__ static Regs load(const State& s, int64_t j) {
    Regs r;
    r.V = s.V[j];
    r.m = s.m[j];
    r.h = s.h[j];
    r.n = s.n[j];
    r.ge = s.ge[j];
    r.gi = s.gi[j];
    return r;
  }
  __device__ static void store(const State& s, int64_t j, const Regs& r) {
    s.V[j] = r.V;
    s.m[j] = r.m;
    s.h[j] = r.h;
    s.n[j] = r.n;
    s.ge[j] = r.ge;
    s.gi[j] = r.gi;
  }
  // The gate updates and channel conductances need only the previous state, so they run
  // before the step's inputs are awaited; the rest of the step follows once they are in.
  static constexpr bool kPrepare = true;
  // HH keeps 11 values per neuron in registers: its 14 parameters and the row pointers stay
  // scalar (in VGPRs they pushed the 4-neuron kernel to 128 VGPRs and 76 bytes of spills;
  // 1M-neuron COBA-HH net 9.86 -> 9.49 us per step without them)
  static constexpr bool kParamVgprs = false;
  // count words published one destination per lane (1M-neuron COBA-HH net 9.48 -> 9.17 us per step;
  // the LIF runner measured 7.21 -> 7.25 with it)
  static constexpr bool kPubByLane = true;
  __device__ static void prepare(const Params& p, Regs& r) {
    r.pre = bs_hh_prepare(p, r.V, r.m, r.h, r.n);
  }
  __device__ static bool update(const Params& p, Regs& r, float in_e, float in_i) {
    return bs_hh_finish(p, r.pre, r.V, r.m, r.h, r.n, r.ge, r.gi, in_e, in_i);
  }
  // No row prefetch for HH: its spikes are rarer and its update is VALU-heavy, and on the
  // 1M-neuron net prefetching the rows of neurons on the upstroke (V within 10-60 mV below
  // threshold) made the step slower, not faster.
  __device__ static bool near(const Params&, const Regs&) { return false; }
};

// Load through a global-memory pointer.  The row pointers are held in VGPRs through an
// empty asm statement, after which the compiler no longer knows their address space and
// would emit flat loads.
template <class T>
__device__ __forceinline__ T ld_global(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

// Synapse row of neuron i (global index) in the E or I connectivity.
struct Row {
  const int32_t* idx;
  const float* w;
  int32_t k;
  bool inh;
};
__device__ __forceinline__ Row row_of(const NetArgs& a, int32_t i) {
  if (i < a.n_exc) {
    const int64_t r = (int64_t)i * a.k_e;
    return Row{a.idx_e + r, a.w_e ? a.w_e + r : nullptr, a.k_e, false};
  }
  const int64_t r = (int64_t)(i - a.n_exc) * a.k_i;
  return Row{a.idx_i + r, a.w_i ? a.w_i + r : nullptr, a.k_i, true};
}

constexpr int kTab = 256;  // repeated-sum table entries per kind (homogeneous weights)

// w added c times in one fp32 chain, from a table of the first kTab partial sums.
__device__ __forceinline__ float repeated_sum(const float* tab, float w, uint32_t c) {
  if (c < (uint32_t)kTab) return tab[c];
  float s = tab[kTab - 1];
  for (uint32_t i = kTab - 1; i < c; ++i) s = s + w;
  return s;
}

// Fixed-point value of a per-synapse weight: rint(w * 2^S) (|w| * 2^S < 2^30 by the choice
// of S, so the conversion is exact).
__device__ __forceinline__ int32_t quantize(float w, float scale) {
  return (int32_t)bs_rint(w * scale);
}

template <class Model, int NPT, bool kHet, int kIn>
__global__ __launch_bounds__(kBlock) void k_run(NetArgs a, typename Model::State st,
                                                typename Model::Params p_arg) {
  // The parameters live in VGPRs (uniform values, one register each) where the model allows:
  // the update reads them as vector operands, so they take no scalar registers in a loop that
  // is short of them.
  typename Model::Params p = p_arg;
  if constexpr (Model::kParamVgprs) {
    static_assert(sizeof(p) % 4 == 0, "parameters are 32-bit words");
    uint32_t* pw = reinterpret_cast<uint32_t*>(&p);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(p) / 4); ++i) asm volatile("" : "+v"(pw[i]));
  }
  constexpr int kChunk = NPT * kBlock;
  static_assert(kChunk < 65536, "a workgroup's E and I spike counts share one 32-bit word");
  constexpr int kBatch = 4;                   // phase A: entry loads in flight per thread
  constexpr int kChunks = 4;                  // phase D: 64-synapse chunks per wave and round
  constexpr int kSlots = NPT >= 8 ? 8 : 16;   // phase D: LDS slots per destination and round
  __shared__ uint32_t s_acc[2 * kChunk];      // input words per neuron: [2 loc] E, [2 loc + 1] I
  __shared__ float s_tab[2][kTab];            // homogeneous: repeated sums of w_e, w_i
  __shared__ uint32_t s_pos[kMaxBlocks];      // next inbox entry per destination (d <- me)
  __shared__ uint64_t s_ofs_in[kMaxBlocks];   // inbox offset (me <- s)
  __shared__ uint32_t s_ofs_out[kMaxBlocks];  // first inbox entry of (d <- me)
  __shared__ int32_t s_list[kChunk];          // this step's spikes: E from the front, I from the back
  __shared__ uint32_t s_nsp[2];               // E | I << 16 spike counts, by step parity
  __shared__ uint32_t s_hash;
  __shared__ uint32_t s_ovf;                  // an entry of this step was stored past the slots
  __shared__ uint32_t s_junk[BS_WAVE];        // destination of the row prefetches (never read)
  __shared__ uint32_t s_rcnt[kMaxBlocks];     // expand round: entries per destination
  __shared__ uint64_t s_stage[kMaxBlocks * kSlots];  // expand round: per-destination slots

  const NetLayout& L = a.L;
  const int nb = L.nb;
  const int me = blockIdx.x;
  const int lane = bs_lane();
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / BS_WAVE);  // wave-uniform
  const int64_t base = (int64_t)me * kChunk;
  const int64_t n = a.n;
  // this thread's neurons jv0 + q * kBlock (n < 2^31: 32-bit), and which of them exist and
  // are excitatory, as bit q of two masks: the same every step, so tested once per launch
  // (a 64-bit compare costs two VALU ops on every lane, and every step used several)
  const uint32_t jv0 = (uint32_t)me * kChunk + threadIdx.x;
  uint32_t valid = 0u, exc = 0u;
#pragma unroll
  for (int q = 0; q < NPT; ++q) {
    valid |= (jv0 + q * kBlock < (uint32_t)a.n ? 1u : 0u) << q;
    exc |= (jv0 + q * kBlock < (uint32_t)a.n_exc ? 1u : 0u) << q;
  }
  WsHeader* hdr = (WsHeader*)a.ws;
  uint64_t* cnt = (uint64_t*)(a.ws + L.off_cnt);
  const uint64_t* ofs = (const uint64_t*)(a.ws + L.off_ofs);
  char* inbox = a.ws + L.off_inbox;
  const size_t buf_bytes = (size_t)L.total * L.entry;

  for (int s = threadIdx.x; s < nb; s += kBlock) {
    s_ofs_in[s] = ofs[(int64_t)me * nb + s];
    s_ofs_out[s] = (uint32_t)ofs[(int64_t)s * nb + me];  // entry counts are < 2^32
    s_pos[s] = s_ofs_out[s];
    s_rcnt[s] = 0;
  }
  for (int i = threadIdx.x; i < 2 * kChunk; i += kBlock) s_acc[i] = 0u;
  // per-synapse weights: 2^S and 2^-S per kind; homogeneous: the repeated-sum tables
  float qscale[2] = {1.0f, 1.0f}, qinv[2] = {1.0f, 1.0f};
  if (kHet) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int S = __builtin_amdgcn_readfirstlane(hdr->qexp[k]);
      qscale[k] = bs_pow2i(S);
      qinv[k] = bs_pow2i(-S);
      asm volatile("" : "+v"(qscale[k]), "+v"(qinv[k]));
    }
  } else if (threadIdx.x == 0 || threadIdx.x == BS_WAVE) {
    const int k = threadIdx.x == 0 ? 0 : 1;
    const float w = k ? a.w_i_homo : a.w_e_homo;
    float s = 0.0f;
    s_tab[k][0] = 0.0f;
    for (int c = 1; c < kTab; ++c) {
      s = s + w;
      s_tab[k][c] = s;
    }
  }

  typename Model::Regs r[NPT];
  // kIn: 0 the parameters' I_ext, 1 each neuron's own (read once per launch), 2 each step's
  float iext[NPT];  // kIn == 1: each neuron's external input
#pragma unroll
  for (int q = 0; q < NPT; ++q) {
    const int64_t j = base + q * kBlock + threadIdx.x;
    iext[q] = 0.0f;
    if (j < n) {
      r[q] = Model::load(st, j);
      if constexpr (kIn == 1) iext[q] = a.iext[j];
    }
  }
  bool last[NPT];
#pragma unroll
  for (int q = 0; q < NPT; ++q) last[q] = false;
  // chunk slots per E / I spike: 64-synapse chunks of its row, rounded up to a power of two
  int lgE = 0, lgI = 0;
  while ((BS_WAVE << lgE) < a.k_e) ++lgE;
  while ((BS_WAVE << lgI) < a.k_i) ++lgI;
  // values used only in vector arithmetic and addresses: VGPRs, like the parameters
  if constexpr (Model::kParamVgprs) {
    asm volatile("" : "+v"(a.idx_e), "+v"(a.w_e), "+v"(a.idx_i), "+v"(a.w_i));
    asm volatile("" : "+v"(a.n_exc), "+v"(a.k_e), "+v"(a.k_i), "+v"(a.w_e_homo), "+v"(a.w_i_homo));
  }
  if (threadIdx.x == 0) {
    s_nsp[0] = s_nsp[1] = 0;
    s_ovf = 0u;
    s_hash = 0;
  }
  int tps = 1;  // threads per source in phase A (power of two, tps * nb <= kBlock)
  while (tps * 2 * nb <= kBlock) tps *= 2;
  const int ring = L.ring;
  const int64_t dly = L.delay;
  int slot_rd = a.slot_rd, slot_wr = a.slot_wr;  // advance by one slot per step
  // a per-step input: step t's value, loaded during step t - 1 (at the start of its phase A,
  // beside the count-word polls, so no wait is added for it)
  float I_cur = 0.0f, I_next = 0.0f;
  if constexpr (kIn == 2) I_cur = ld_input(a.isched);
  __syncthreads();

  for (int32_t t = 0; t < a.steps; ++t) {
    const int64_t ta = a.t0 + t;  // absolute step index
    if constexpr (kIn == 2) p.I_ext = I_cur;

    // ---- prefetch: synapse rows of neurons that may spike this step, into L2 ----
    // Issued before the waits of phase A, whose loads wait for them anyway, so they cost no
    // latency; the expand phase then finds most spiking rows in L2 instead of HBM.  The
    // loads write to LDS (s_junk) rather than registers, so no register is held for them.
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      if (((valid >> q) & 1u) && Model::near(kIn == 1 ? with_input(p, iext[q]) : p, r[q])) {
        int32_t jv = (int32_t)(jv0 + q * kBlock);
        asm volatile("" : "+v"(jv));  // keeps the row addresses from being hoisted out of the loop
        const Row rw = row_of(a, jv);
        const int last = rw.k - 1;
        if (last >= 0) {
#pragma unroll
          for (int u = 0; u < 5; ++u) {  // every 128-byte line of the first 128 synapses + the last
            const int o = (u < 4 && u * 32 < last) ? u * 32 : last;
            __builtin_amdgcn_global_load_lds((const void*)(rw.idx + o), (void*)s_junk, 4, 0, 0);
            if (kHet)
              __builtin_amdgcn_global_load_lds((const void*)(rw.w + o), (void*)s_junk, 4, 0, 0);
          }
        }
      }
    }

    // ---- A: inputs produced by step ta-1-D ----
    // tps threads per source: all poll the source's count word (one transaction per
    // wave), then each reads every tps-th entry, up to kBatch loads in flight per thread.
    // The first look at each count word is issued before the input-independent part of the
    // update (Model::prepare), which runs while those loads are in flight.
    const uint64_t* cin = cnt + ((int64_t)slot_rd * nb + me) * nb;
    if constexpr (kIn == 2) {
      if (t + 1 < a.steps) I_next = ld_input(a.isched + t + 1);
    }
    uint64_t v_first = 0;
    if (Model::kPrepare) {
      if (ta > dly && (int)threadIdx.x < nb * tps) v_first = ld_dev64(cin + threadIdx.x / tps);
#pragma unroll
      for (int q = 0; q < NPT; ++q) {
        if (base + q * kBlock + threadIdx.x < n) Model::prepare(p, r[q]);
      }
    }
    if (ta > dly) {
      const uint32_t want = (uint32_t)(ta - dly);  // step u publishes tag u + 1
      const char* ib = inbox + (size_t)slot_rd * buf_bytes;
      for (int x = threadIdx.x; x < nb * tps; x += kBlock) {
        const int s = x / tps;
        const uint32_t sub = (uint32_t)(x - s * tps);
        uint64_t v = (Model::kPrepare && x == (int)threadIdx.x) ? v_first : ld_dev64(cin + s);
        uint64_t spins = 0;
        while ((uint32_t)(v >> 32) != want) {
          if (++spins > kSpinLimit) {
            st_dev32(&hdr->error, 1u);
            v = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(BS_POLL_SLEEP);
          v = ld_dev64(cin + s);
        }
        const uint32_t c = (uint32_t)v;
        const uint64_t o = s_ofs_in[s];
        for (uint32_t e0 = sub; e0 < c; e0 += kBatch * tps) {
          uint64_t ent[kBatch];
#pragma unroll
          for (int u = 0; u < kBatch; ++u) {
            const uint32_t e = e0 + u * tps;
            ent[u] = 0;
            if (e < c) {
              if (kHet) ent[u] = ld_dev64((const uint64_t*)ib + o + e);
              else ent[u] = ld_dev32((const uint32_t*)ib + o + e) | (1ull << 32);
            }
          }
#pragma unroll
          for (int u = 0; u < kBatch; ++u) {
            if (e0 + u * tps < c) {
              const uint32_t tgt = (uint32_t)ent[u];
              // per-synapse: the fixed-point weight (two's complement); homogeneous: one event
              const uint32_t add = kHet ? (uint32_t)(ent[u] >> 32) : 1u;
              const uint32_t loc = tgt & ~kInhFlag;
              if (loc < (uint32_t)kChunk)
                atomicAdd(&s_acc[2 * loc + ((tgt & kInhFlag) ? 1 : 0)], add);
            }
          }
        }
      }
      __syncthreads();
    }

    // ---- B: fused update ----
    uint32_t h = 0;
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int loc = q * kBlock + threadIdx.x;
      last[q] = false;
      if ((valid >> q) & 1u) {
        const uint2 acc = *(uint2*)&s_acc[2 * loc];
        *(uint2*)&s_acc[2 * loc] = make_uint2(0u, 0u);
        float in_e, in_i;
        if (kHet) {
          in_e = (float)(int32_t)acc.x * qinv[0];
          in_i = (float)(int32_t)acc.y * qinv[1];
        } else {
          in_e = repeated_sum(s_tab[0], a.w_e_homo, acc.x);
          in_i = repeated_sum(s_tab[1], a.w_i_homo, acc.y);
        }
        last[q] = Model::update(kIn == 1 ? with_input(p, iext[q]) : p, r[q], in_e, in_i);
        if (last[q]) h += bs_mix32(jv0 + q * kBlock);
        if (a.raster) a.raster[(int64_t)t * n + (jv0 + q * kBlock)] = last[q] ? 1 : 0;
      }
    }

    // ---- C: block list of this step's spikes ----
    // E spikes fill s_list from the front and I spikes from the back; each wave reserves its
    // two ranges with one LDS atomic on a word holding both counts (at most 8192 each: no
    // carry between the halves), no scan, one barrier.  One atomic per wave instead of one
    // per kind: 7.20 -> 7.16 us per step for the 1M-neuron COBA-LIF net.
    uint32_t* nsp2 = &s_nsp[ta & 1];  // this step's E spikes (bits 0-15), I spikes (16-31)
    {
      uint64_t mE[NPT], mI[NPT];
      uint32_t wE = 0, wI = 0;
#pragma unroll
      for (int q = 0; q < NPT; ++q) {
        const bool e = (exc >> q) & 1u;
        mE[q] = bs_ballot(last[q] && e);
        mI[q] = bs_ballot(last[q] && !e);
        wE += (uint32_t)__popcll(mE[q]);
        wI += (uint32_t)__popcll(mI[q]);
      }
      uint32_t b = 0;
      if (lane == 0 && (wE | wI)) b = atomicAdd(nsp2, wE | (wI << 16));
      b = __builtin_amdgcn_readfirstlane(b);
      uint32_t bE = b & 0xFFFFu, bI = b >> 16;
#pragma unroll
      for (int q = 0; q < NPT; ++q) {
        const int32_t j = (int32_t)(jv0 + q * kBlock);
        if (last[q]) {
          if ((exc >> q) & 1u) s_list[bE + bs_rank_below(mE[q])] = j;
          else s_list[kChunk - 1 - (int)(bI + bs_rank_below(mI[q]))] = j;
        }
        bE += (uint32_t)__popcll(mE[q]);
        bI += (uint32_t)__popcll(mI[q]);
      }
    }
    if (h) atomicAdd(&s_hash, h);
    __syncthreads();
    if (threadIdx.x == 0) {  // per-workgroup partials, summed over workgroups after the launch
      if (a.counts) a.counts[(int64_t)t * nb + me] = (*nsp2 & 0xFFFFu) + (*nsp2 >> 16);
      if (a.hash) a.hash[(int64_t)t * nb + me] = s_hash;
      // s_hash's last reader; the next adds come after this step's final barrier
      s_hash = 0;
    }

    // ---- D: expand spikes into the destinations' inboxes ----
    // Each spike's row is cut into 64-synapse chunks (cpE / cpI chunk slots per E / I spike,
    // a power of two); chunk g goes to wave g % 16, up to kChunks per wave and round.  Lane l
    // of a chunk loads synapse c*64 + l of the row (the row address is wave-uniform), takes a
    // rank among this round's entries for the destination from an LDS counter and parks the
    // entry in the destination's kSlots LDS slots (entries past them are stored directly).
    // After one barrier the slots are written out destination by destination, so consecutive
    // lanes store to consecutive inbox addresses, and each destination's cursor advances.
    char* ob = inbox + (size_t)slot_wr * buf_bytes;
    const uint32_t nEI = __builtin_amdgcn_readfirstlane(*nsp2);
    const uint32_t nE = nEI & 0xFFFFu, nI = nEI >> 16;
    const uint32_t gE = nE << lgE;
    const uint32_t G = gE + (nI << lgI);
    constexpr uint32_t kPer = kWaves * kChunks;
    const uint32_t rounds = (G + kPer - 1) / kPer;
    for (uint32_t rnd = 0; rnd < rounds; ++rnd) {
      // all chunk loads of the round are issued before any of them is used
      int32_t tgt[kChunks];
      float wraw[kChunks];  // per-synapse weights only
      bool inh[kChunks];
#pragma unroll
      for (int u = 0; u < kChunks; ++u) {
        tgt[u] = -1;
        wraw[u] = 0.0f;
        inh[u] = false;
        const uint32_t g = rnd * kPer + (uint32_t)(u * kWaves + wid);
        if (g < G) {
          int32_t jw;
          uint32_t c;
          if (g < gE) {
            jw = s_list[g >> lgE];
            c = g & ((1u << lgE) - 1u);
          } else {
            const uint32_t g2 = g - gE;
            jw = s_list[kChunk - 1 - (int)(g2 >> lgI)];
            c = g2 & ((1u << lgI) - 1u);
          }
          jw = __builtin_amdgcn_readfirstlane(jw);
          const Row rw = row_of(a, jw);
          const int32_t tt = (int32_t)(c * BS_WAVE) + lane;
          if (tt < rw.k) {
            tgt[u] = ld_global(rw.idx + tt);
            if (kHet) wraw[u] = ld_global(rw.w + tt);
            inh[u] = rw.inh;
          }
        }
      }
      int32_t wq[kChunks];  // fixed-point weights
#pragma unroll
      for (int u = 0; u < kChunks; ++u)
        wq[u] = kHet ? quantize(wraw[u], inh[u] ? qscale[1] : qscale[0]) : 0;
#pragma unroll
      for (int u = 0; u < kChunks; ++u) {
        if ((uint32_t)tgt[u] < (uint32_t)n) {
          const int d = tgt[u] >> L.shift;
          const uint32_t rk = atomicAdd(&s_rcnt[d], 1u);
          const uint32_t loc = (uint32_t)(tgt[u] & (kChunk - 1)) | (inh[u] ? kInhFlag : 0u);
          const uint64_t ent =
              kHet ? (((uint64_t)(uint32_t)wq[u] << 32) | loc) : (uint64_t)loc;
          if (rk < (uint32_t)kSlots) {
            s_stage[d * kSlots + rk] = ent;
          } else {  // slots full: store this one directly
            s_ovf = 1u;
            const uint32_t pos = s_pos[d] + rk;
            if (kHet) st_dev64((uint64_t*)ob + pos, ent);
            else st_dev32((uint32_t*)ob + pos, (uint32_t)ent);
          }
        }
      }
      __syncthreads();
      // write-out: kSlots consecutive lanes per destination (all in one wave), then the
      // destination's first lane advances its cursor and clears its round count
      for (int x = threadIdx.x; x < nb * kSlots; x += kBlock) {
        const int d = x / kSlots;
        const uint32_t slot = (uint32_t)(x - d * kSlots);
        // one LDS round trip: the round count, the cursor and the slot (read even when
        // empty), the cursor reused for its advance (7.24 -> 7.19 us per step for the 1M-neuron COBA-LIF net)
        const uint32_t rc = s_rcnt[d];
        const uint32_t p0 = s_pos[d];
        uint64_t ent = s_stage[x];
        asm volatile("" : "+v"(ent));  // keeps the read beside the other two
        if (slot < rc) {
          if (kHet) st_dev64((uint64_t*)ob + p0 + slot, ent);
          else st_dev32((uint32_t*)ob + p0 + slot, (uint32_t)ent);
        }
        if (slot == 0 && rc) {
          s_pos[d] = p0 + rc;
          s_rcnt[d] = 0;
        }
      }
      if (rnd + 1 < rounds) __syncthreads();  // slots and round counts are reused
    }
    // read before the wait, so that no LDS access follows it before the first publication
    const bool ovf = rounds > 0 && s_ovf != 0u;   // uniform: set before the round barrier
    __builtin_amdgcn_s_waitcnt(0);  // this wave's entries are complete at device scope
    // Destination d's staged entries were all written by the wave of write-out slots
    // [d*kSlots, (d+1)*kSlots), so that wave alone publishes d once its own stores are
    // complete -- unless an entry went past the slots (stored by another wave): then every
    // wave's stores are awaited first.
    if (ovf) __syncthreads();
    {
      uint64_t* cout = cnt + (int64_t)slot_wr * nb * nb;
      const uint64_t tag = (uint64_t)(uint32_t)(ta + 1) << 32;
      if constexpr (Model::kPubByLane) {
        // the wave's destinations (kSpw per write-out iteration), one lane each: one LDS
        // round trip instead of one per iteration
        constexpr int kSpw = BS_WAVE / kSlots;   // destinations per wave and iteration
        constexpr int kDpi = kBlock / kSlots;    // destinations per iteration
        constexpr int kPubLanes = kSpw * ((kMaxBlocks + kDpi - 1) / kDpi);
        static_assert(kPubLanes <= BS_WAVE, "one lane per destination of the wave");
        const int d = (lane / kSpw) * kDpi + wid * kSpw + lane % kSpw;
        if (lane < kPubLanes && d < nb) {
          const uint32_t o0 = s_ofs_out[d];
          st_dev64(cout + (int64_t)d * nb + me, tag | (s_pos[d] - o0));
          s_pos[d] = o0;
        }
      } else {
        for (int x = threadIdx.x; x < nb * kSlots; x += kBlock) {
          if (x % kSlots) continue;
          const int d = x / kSlots;
          st_dev64(cout + (int64_t)d * nb + me, tag | (s_pos[d] - s_ofs_out[d]));
          s_pos[d] = s_ofs_out[d];
        }
      }
      if (ovf) {
        __syncthreads();
        if (threadIdx.x == 0) s_ovf = 0u;
      }
      // Clear the counters this step used: every read of them came before the barrier
      // above, and their next user is step ta+2, whose adds follow step ta+1's final
      // barrier.  (Clearing the other parity here would race with step ta+1's adds when
      // phase A has no barrier, i.e. while ta+1 <= D.)
      if (threadIdx.x == 0) s_nsp[ta & 1] = 0;
    }
    slot_rd = slot_rd + 1 == ring ? 0 : slot_rd + 1;
    slot_wr = slot_wr + 1 == ring ? 0 : slot_wr + 1;
    if constexpr (kIn == 2) I_cur = I_next;
  }

#pragma unroll
  for (int q = 0; q < NPT; ++q) {
    const int64_t j = base + q * kBlock + threadIdx.x;
    if (j < n) {
      Model::store(st, j, r[q]);
      if (a.steps > 0) a.spk[j] = last[q] ? 1 : 0;
    }
  }
}

// ---- seeding: a spike vector published as the events of step t0 - 1 ----
// For a run that starts from a state with pending spikes (a loop handed over after some
// steps elsewhere): workgroup s expands the spikes of its slice into its inboxes of ring
// slot a.slot_wr, exactly as phase D of k_run would, and publishes every destination's count
// word with the tag of step t0 - 1.  Synaptic delay 0 only.  Workgroups do not wait on one
// another: plain launch.
template <bool kHet>
__global__ __launch_bounds__(kBlock) void k_seed(NetArgs a, const uint8_t* spk0, uint32_t tag) {
  __shared__ uint32_t s_cnt[kMaxBlocks];
  const NetLayout& L = a.L;
  const int nb = L.nb;
  const int me = blockIdx.x;
  const int lane = bs_lane();
  const int wid = threadIdx.x / BS_WAVE;
  const WsHeader* hdr = (const WsHeader*)a.ws;
  uint64_t* cnt = (uint64_t*)(a.ws + L.off_cnt);
  const uint64_t* ofs = (const uint64_t*)(a.ws + L.off_ofs);
  char* ob = a.ws + L.off_inbox + (size_t)a.slot_wr * (size_t)L.total * L.entry;
  for (int d = threadIdx.x; d < nb; d += kBlock) s_cnt[d] = 0u;
  float qscale[2] = {1.0f, 1.0f};
  if (kHet) {
    qscale[0] = bs_pow2i(hdr->qexp[0]);
    qscale[1] = bs_pow2i(hdr->qexp[1]);
  }
  __syncthreads();
  const int64_t chunk = (int64_t)1 << L.shift;
  const int64_t lo = (int64_t)me * chunk;
  const int64_t hi = lo + chunk < a.n ? lo + chunk : a.n;
  for (int64_t i = lo + wid; i < hi; i += kWaves) {  // one row per wave and iteration
    if (spk0[i] == 0) continue;
    const Row rw = row_of(a, (int32_t)i);
    for (int tt = lane; tt < rw.k; tt += BS_WAVE) {
      const int32_t tgt = rw.idx[tt];
      if ((uint32_t)tgt >= (uint32_t)a.n) continue;
      const int d = tgt >> L.shift;
      const uint32_t rk = atomicAdd(&s_cnt[d], 1u);
      const uint32_t loc = (uint32_t)(tgt & (chunk - 1)) | (rw.inh ? kInhFlag : 0u);
      const uint32_t pos = (uint32_t)ofs[(int64_t)d * nb + me] + rk;
      if (kHet)
        st_dev64((uint64_t*)ob + pos,
                 ((uint64_t)(uint32_t)quantize(rw.w[tt], rw.inh ? qscale[1] : qscale[0]) << 32) |
                     loc);
      else
        st_dev32((uint32_t*)ob + pos, loc);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's entries are complete at device scope
  __syncthreads();
  uint64_t* cout = cnt + (int64_t)a.slot_wr * nb * nb;
  for (int d = threadIdx.x; d < nb; d += kBlock)
    st_dev64(cout + (int64_t)d * nb + me, ((uint64_t)tag << 32) | s_cnt[d]);
}

// ---- setup: per-(source, destination) capacities and inbox offsets ----

__global__ __launch_bounds__(kBlock) void k_caps(NetArgs a, uint32_t* cap) {
  __shared__ uint32_t hist[kMaxBlocks];
  const int nb = a.L.nb;
  const int me = blockIdx.x;
  for (int d = threadIdx.x; d < nb; d += kBlock) hist[d] = 0;
  __syncthreads();
  const int64_t chunk = (int64_t)1 << a.L.shift;
  const int64_t lo = (int64_t)me * chunk;
  const int64_t hi = lo + chunk < a.n ? lo + chunk : a.n;
  // kRows rows per wave at a time, lane l reading synapse l (+ 64 j) of each, their loads in
  // flight together (one row per workgroup and iteration waited ~1 us per row: ~4 ms for the
  // 4,096-row slices of a 1M-neuron net)
  constexpr int kRows = 4;
  const int lane = bs_lane();
  const int wid = threadIdx.x / BS_WAVE;
  for (int64_t i0 = lo + (int64_t)wid * kRows; i0 < hi; i0 += (int64_t)kWaves * kRows) {
    Row rw[kRows];
    int32_t kmax = 0;
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      rw[u] = i0 + u < hi ? row_of(a, (int32_t)(i0 + u)) : Row{nullptr, nullptr, 0, false};
      kmax = rw[u].k > kmax ? rw[u].k : kmax;
    }
    for (int32_t t0 = 0; t0 < kmax; t0 += BS_WAVE) {
      int32_t tgt[kRows];
#pragma unroll
      for (int u = 0; u < kRows; ++u) tgt[u] = t0 + lane < rw[u].k ? rw[u].idx[t0 + lane] : -1;
#pragma unroll
      for (int u = 0; u < kRows; ++u)
        if ((uint32_t)tgt[u] < (uint32_t)a.n) atomicAdd(&hist[tgt[u] >> a.L.shift], 1u);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < nb; d += kBlock) cap[(int64_t)me * nb + d] = hist[d];
}

// Exclusive scan of cap in destination-major order -> ofs[d][s]; one workgroup.
__global__ __launch_bounds__(kBlock) void k_offsets(int nb, const uint32_t* cap, uint64_t* ofs,
                                                    uint64_t* total) {
  __shared__ uint64_t part[kBlock];
  const int64_t m = (int64_t)nb * nb;
  const int64_t per = (m + kBlock - 1) / kBlock;
  const int64_t lo = threadIdx.x * per;
  const int64_t hi = lo + per < m ? lo + per : m;
  uint64_t sum = 0;
  for (int64_t x = lo; x < hi; ++x) {  // x = d*nb + s
    const int64_t d = x / nb, s = x - d * nb;
    sum += cap[s * nb + d];
  }
  part[threadIdx.x] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t acc = 0;
    for (int i = 0; i < kBlock; ++i) {
      const uint64_t v = part[i];
      part[i] = acc;
      acc += v;
    }
    *total = acc;
  }
  __syncthreads();
  uint64_t acc = part[threadIdx.x];
  for (int64_t x = lo; x < hi; ++x) {
    const int64_t d = x / nb, s = x - d * nb;
    ofs[x] = acc;
    acc += cap[s * nb + d];
  }
}

// Per-synapse weights: in-degree of every neuron per kind (valid targets) and the bit
// pattern of max |w| per kind (all weights of the kind).
__global__ __launch_bounds__(256) void k_indeg(NetArgs a, uint32_t* deg, WsHeader* hdr) {
  const int64_t tot_e = (int64_t)a.n_exc * a.k_e;
  const int64_t tot = tot_e + (int64_t)(a.n - a.n_exc) * a.k_i;
  uint32_t wb[2] = {0u, 0u};
  for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < tot;
       s += (int64_t)gridDim.x * blockDim.x) {
    const int k = s >= tot_e ? 1 : 0;
    const int64_t o = k ? s - tot_e : s;
    const int32_t tgt = k ? a.idx_i[o] : a.idx_e[o];
    const uint32_t b = __float_as_uint(k ? a.w_i[o] : a.w_e[o]) & 0x7FFFFFFFu;
    wb[k] = b > wb[k] ? b : wb[k];
    if ((uint32_t)tgt < (uint32_t)a.n) atomicAdd(&deg[(int64_t)k * a.n + tgt], 1u);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    uint32_t m = wb[k];
    for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
      const uint32_t v = __shfl_xor(m, o);
      m = v > m ? v : m;
    }
    if (bs_lane() == 0 && m) atomicMax(&hdr->wbits[k], m);
  }
}

// S per kind from D = max in-degree and W = max |w|: with W < 2^e_w and D <= 2^e_d,
// S = 30 - e_w - e_d (at most 100) keeps |sum of rounded weights| < 2^30 + D/2 < 2^31.
// A weight that is not finite, or S < -100, sets error 2.  One workgroup.
__global__ __launch_bounds__(kBlock) void k_qexp(int32_t n, const uint32_t* deg, WsHeader* hdr) {
  __shared__ uint32_t s_max[2][kWaves];
  uint32_t m[2] = {0u, 0u};
  for (int64_t j = threadIdx.x; j < n; j += kBlock) {
    const uint32_t de = deg[j], di = deg[(int64_t)n + j];
    m[0] = de > m[0] ? de : m[0];
    m[1] = di > m[1] ? di : m[1];
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
      const uint32_t v = __shfl_xor(m[k], o);
      m[k] = v > m[k] ? v : m[k];
    }
    if (bs_lane() == 0) s_max[k][threadIdx.x / BS_WAVE] = m[k];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 0; k < 2; ++k) {
      uint32_t D = 0;
      for (int w = 0; w < kWaves; ++w) D = s_max[k][w] > D ? s_max[k][w] : D;
      const uint32_t wb = hdr->wbits[k];
      const int e_w = (wb >> 23) ? (int)(wb >> 23) - 126 : -126;
      const int e_d = D <= 1 ? 0 : 32 - __clz(D - 1);
      int S = 30 - e_w - e_d;
      if (S > 100) S = 100;
      if (wb >= 0x7F800000u || S < -100) {
        hdr->error = 2u;
        S = 0;
      }
      hdr->qexp[k] = S;
    }
  }
}

__global__ void k_zero_u64(uint64_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0ull;
}

// counts[t] = sum over workgroups of pc[t][b]; hash[t] likewise (mod 2^32).  One wave per step.
__global__ void k_sum_parts(int nb, int32_t steps, const uint32_t* pc, const uint32_t* ph,
                            int32_t* counts, uint32_t* hash) {
  const int32_t t = blockIdx.x * 4 + threadIdx.x / BS_WAVE;
  const int lane = threadIdx.x % BS_WAVE;
  if (t >= steps) return;
  uint32_t c = 0, h = 0;
  for (int b = lane; b < nb; b += BS_WAVE) {
    if (counts) c += pc[(int64_t)t * nb + b];
    if (hash) h += ph[(int64_t)t * nb + b];
  }
  for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
    c += __shfl_xor(c, o);
    h += __shfl_xor(h, o);
  }
  if (lane == 0) {
    if (counts) counts[t] = (int32_t)c;
    if (hash) hash[t] = h;
  }
}

// ---- host helpers ----

int npt_for(int64_t n, int64_t threads) {
  const int64_t need = (n + threads - 1) / threads;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  return -1;
}

int ilog2(int64_t x) {
  int s = 0;
  while (((int64_t)1 << s) < x) ++s;
  return s;
}

// Workgroup count and slice size: as few neurons per thread as the grid allows.
int plan(const bs_net* net, NetLayout* L) {
  const int cus = bs_num_cus();
  const int bpc = net->blocks_per_cu > 0 ? net->blocks_per_cu : 1;
  int64_t grid = (int64_t)bpc * cus;
  if (grid > kMaxBlocks) grid = kMaxBlocks;
  const int npt = npt_for(net->n, grid * kBlock);
  if (npt < 0) return -1;
  const int64_t chunk = (int64_t)npt * kBlock;
  int64_t nb = (net->n + chunk - 1) / chunk;
  if (nb < 1) nb = 1;
  L->nb = (int32_t)nb;
  L->npt = npt;
  L->shift = ilog2(chunk);
  L->entry = net->w_e ? 8u : 4u;
  // worst case: every synapse delivers one entry (invalid targets are never stored)
  L->total = (uint64_t)net->n_exc * (uint64_t)net->k_e +
             (uint64_t)(net->n - net->n_exc) * (uint64_t)net->k_i;
  if (L->total >= ((uint64_t)1 << 32)) return -1;  // inbox positions are 32-bit
  L->delay = net->delay_steps;
  L->ring = 2 * (net->delay_steps + 1);
  size_t o = align256(sizeof(WsHeader));
  L->off_cnt = o;
  o = align256(o + (size_t)L->ring * nb * nb * sizeof(uint64_t));
  L->off_cap = o;
  o = align256(o + (size_t)nb * nb * sizeof(uint32_t));
  L->off_ofs = o;
  o = align256(o + (size_t)(nb * nb + 1) * sizeof(uint64_t));
  L->off_part = o;
  o = align256(o + (size_t)2 * kRunSteps * nb * sizeof(uint32_t));
  L->off_deg = o;
  if (net->w_e) o = align256(o + (size_t)2 * net->n * sizeof(uint32_t));
  L->off_vprev = o;
  o = align256(o + (size_t)net->n * sizeof(float));
  L->off_inbox = o;
  o = align256(o + (size_t)L->ring * L->total * L->entry);
  L->bytes = o;
  return 0;
}

int check_net(const bs_net* net, const char* who) {
  BS_CHECK_ARG(net != nullptr, "%s: net is NULL", who);
  BS_CHECK_ARG(net->n > 0 && net->n_exc >= 0 && net->n_exc <= net->n,
               "%s: bad sizes n=%d n_exc=%d", who, net->n, net->n_exc);
  BS_CHECK_ARG(net->k_e >= 0 && net->k_i >= 0, "%s: negative fan-out", who);
  BS_CHECK_ARG(net->spk != nullptr, "%s: spk is NULL", who);
  BS_CHECK_ARG(net->n_exc == 0 || net->k_e == 0 || net->idx_e, "%s: idx_e is NULL", who);
  BS_CHECK_ARG(net->n_exc == net->n || net->k_i == 0 || net->idx_i, "%s: idx_i is NULL", who);
  BS_CHECK_ARG((net->w_e == nullptr) == (net->w_i == nullptr),
               "%s: w_e and w_i must both be given or both be NULL", who);
  BS_CHECK_ARG(net->delay_steps >= 0 && net->delay_steps <= kMaxDelay,
               "%s: delay_steps=%d outside [0, %d]", who, net->delay_steps, kMaxDelay);
  return BS_OK;
}

NetArgs make_args(const bs_net* net, const NetLayout& L, void* ws) {
  NetArgs a;
  a.n = net->n;
  a.n_exc = net->n_exc;
  a.k_e = net->k_e;
  a.k_i = net->k_i;
  a.idx_e = net->idx_e;
  a.w_e = net->w_e;
  a.w_e_homo = net->w_e_homo;
  a.idx_i = net->idx_i;
  a.w_i = net->w_i;
  a.w_i_homo = net->w_i_homo;
  a.spk = net->spk;
  a.t0 = 0;
  a.steps = 0;
  a.slot_rd = 0;
  a.slot_wr = 0;
  a.counts = nullptr;
  a.hash = nullptr;
  a.raster = nullptr;
  a.iext = net->I_ext;
  a.isched = nullptr;
  a.ws = (char*)ws;
  a.L = L;
  return a;
}

template <class Model, int NPT, bool kHet, int kIn>
int launch_one(const NetArgs& a, const typename Model::State& st, const typename Model::Params& p,
               hipStream_t s) {
  int occ = 0;
  BS_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_run<Model, NPT, kHet, kIn>,
                                                            kBlock, 0));
  if ((int64_t)occ * bs_num_cus() < a.L.nb) {
    bs_set_error("runner: %d workgroups cannot be co-resident (occupancy %d x %d CUs)", a.L.nb,
                 occ, bs_num_cus());
    return BS_ERR_UNSUPPORTED;
  }
  NetArgs aa = a;
  typename Model::State ss = st;
  typename Model::Params pp = p;
  void* args[] = {(void*)&aa, (void*)&ss, (void*)&pp};
  BS_CHECK_HIP(hipLaunchCooperativeKernel((const void*)k_run<Model, NPT, kHet, kIn>, dim3(a.L.nb),
                                          dim3(kBlock), args, 0, s));
  return BS_OK;
}

template <class Model, bool kHet, int kIn>
int dispatch_npt(const NetArgs& a, const typename Model::State& st,
                 const typename Model::Params& p, hipStream_t s) {
  switch (a.L.npt) {
    case 1: return launch_one<Model, 1, kHet, kIn>(a, st, p, s);
    case 2: return launch_one<Model, 2, kHet, kIn>(a, st, p, s);
    case 4: return launch_one<Model, 4, kHet, kIn>(a, st, p, s);
    case 8: return launch_one<Model, 8, kHet, kIn>(a, st, p, s);
  }
  bs_set_error("runner: unsupported neurons-per-thread %d", a.L.npt);
  return BS_ERR_UNSUPPORTED;
}

template <class Model>
int run(const bs_net* net, const typename Model::State* st, const typename Model::Params* p,
        int64_t t0, int32_t steps, int32_t* counts_out, uint32_t* hash_out, uint8_t* raster_out,
        void* workspace, bs_stream_t stream, const char* who, const float* isched = nullptr) {
  int rc = check_net(net, who);
  if (rc) return rc;
  BS_CHECK_ARG(st && p && workspace, "%s: NULL state/params/workspace", who);
  BS_CHECK_ARG(steps >= 0, "%s: steps=%d < 0", who, steps);
  BS_CHECK_ARG(t0 >= 0 && t0 + steps < ((int64_t)1 << 32) - 1, "%s: step index out of range",
               who);
  if (steps == 0) return BS_OK;
  NetLayout L;
  if (plan(net, &L)) {
    bs_set_error("%s: n=%d needs more than %d neurons per thread", who, net->n, kMaxNpt);
    return BS_ERR_UNSUPPORTED;
  }
  hipStream_t s = bs_stream(stream);
  uint32_t* part = (uint32_t*)((char*)workspace + L.off_part);
  // Launches of at most kRunSteps steps; after each, the per-workgroup partials of every
  // step are summed into counts_out / hash_out (plain stores in the kernel instead of one
  // same-address atomic per workgroup and step).
  for (int32_t done = 0; done < steps;) {
    const int32_t len = steps - done < kRunSteps ? steps - done : kRunSteps;
    NetArgs a = make_args(net, L, workspace);
    a.t0 = t0 + done;
    a.steps = len;
    const int64_t R = L.ring;
    a.slot_wr = (int32_t)(a.t0 % R);
    a.slot_rd = (int32_t)(((a.t0 - 1 - L.delay) % R + R) % R);
    a.counts = counts_out ? part : nullptr;
    a.hash = hash_out ? part + (size_t)kRunSteps * L.nb : nullptr;
    a.raster = raster_out ? raster_out + (int64_t)done * net->n : nullptr;
    a.isched = isched ? isched + done : nullptr;
    if (isched)
      rc = net->w_e != nullptr ? dispatch_npt<Model, true, 2>(a, *st, *p, s)
                               : dispatch_npt<Model, false, 2>(a, *st, *p, s);
    else if (net->I_ext)
      rc = net->w_e != nullptr ? dispatch_npt<Model, true, 1>(a, *st, *p, s)
                               : dispatch_npt<Model, false, 1>(a, *st, *p, s);
    else
      rc = net->w_e != nullptr ? dispatch_npt<Model, true, 0>(a, *st, *p, s)
                               : dispatch_npt<Model, false, 0>(a, *st, *p, s);
    if (rc) return rc;
    if (counts_out || hash_out) {
      k_sum_parts<<<(len + 3) / 4, 256, 0, s>>>(L.nb, len, a.counts, a.hash,
                                                counts_out ? counts_out + done : nullptr,
                                                hash_out ? hash_out + done : nullptr);
      BS_CHECK_LAUNCH();
    }
    done += len;
  }
  return BS_OK;
}

}  // namespace

extern "C" size_t bs_net_workspace_size(const bs_net* net) {
  bs_clear_error();
  if (check_net(net, "bs_net_workspace_size")) return 0;
  NetLayout L;
  if (plan(net, &L)) {
    bs_set_error("bs_net_workspace_size: n=%d too large for the grid", net->n);
    return 0;
  }
  return L.bytes;
}

extern "C" int bs_net_grid_blocks(const bs_net* net) {
  bs_clear_error();
  if (check_net(net, "bs_net_grid_blocks")) return -1;
  NetLayout L;
  if (plan(net, &L)) {
    bs_set_error("bs_net_grid_blocks: n=%d too large for the grid", net->n);
    return -1;
  }
  return L.nb;
}

extern "C" int bs_net_prepare(const bs_net* net, void* workspace, bs_stream_t stream) {
  bs_clear_error();
  int rc = check_net(net, "bs_net_prepare");
  if (rc) return rc;
  BS_CHECK_ARG(workspace != nullptr, "bs_net_prepare: workspace is NULL");
  NetLayout L;
  if (plan(net, &L)) {
    bs_set_error("bs_net_prepare: n=%d too large for the grid", net->n);
    return BS_ERR_UNSUPPORTED;
  }
  hipStream_t s = bs_stream(stream);
  char* ws = (char*)workspace;
  NetArgs a = make_args(net, L, workspace);
  // header, tagged counts, capacities, offsets and in-degrees are cleared; inboxes need no
  // clearing
  k_zero_u64<<<256, 256, 0, s>>>((uint64_t*)ws, (int64_t)(L.off_inbox / 8));
  BS_CHECK_LAUNCH();
  if (net->w_e) {  // fixed-point exponents of the per-synapse weights
    uint32_t* deg = (uint32_t*)(ws + L.off_deg);
    k_indeg<<<2048, 256, 0, s>>>(a, deg, (WsHeader*)ws);
    BS_CHECK_LAUNCH();
    k_qexp<<<1, kBlock, 0, s>>>(net->n, deg, (WsHeader*)ws);
    BS_CHECK_LAUNCH();
  }
  k_caps<<<L.nb, kBlock, 0, s>>>(a, (uint32_t*)(ws + L.off_cap));
  BS_CHECK_LAUNCH();
  uint64_t* ofs = (uint64_t*)(ws + L.off_ofs);
  k_offsets<<<1, kBlock, 0, s>>>(L.nb, (const uint32_t*)(ws + L.off_cap), ofs,
                                 ofs + (int64_t)L.nb * L.nb);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_net_seed_spikes(const bs_net* net, const uint8_t* spk, int64_t t0,
                                  void* workspace, bs_stream_t stream) {
  bs_clear_error();
  int rc = check_net(net, "bs_net_seed_spikes");
  if (rc) return rc;
  BS_CHECK_ARG(spk != nullptr && workspace != nullptr, "bs_net_seed_spikes: NULL pointer");
  BS_CHECK_ARG(net->delay_steps == 0,
               "bs_net_seed_spikes: pending spikes can be seeded with synaptic delay 0 only "
               "(delay_steps=%d)", net->delay_steps);
  BS_CHECK_ARG(t0 >= 1 && t0 < ((int64_t)1 << 32) - 1, "bs_net_seed_spikes: t0=%lld outside "
               "[1, 2^32 - 1)", (long long)t0);
  NetLayout L;
  if (plan(net, &L)) {
    bs_set_error("bs_net_seed_spikes: n=%d too large for the grid", net->n);
    return BS_ERR_UNSUPPORTED;
  }
  NetArgs a = make_args(net, L, workspace);
  a.slot_wr = (int32_t)((t0 - 1) % L.ring);
  hipStream_t s = bs_stream(stream);
  if (net->w_e)
    k_seed<true><<<L.nb, kBlock, 0, s>>>(a, spk, (uint32_t)t0);
  else
    k_seed<false><<<L.nb, kBlock, 0, s>>>(a, spk, (uint32_t)t0);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

namespace {

// Deferred reset around a run (bs_lif_params.deferred_reset): the state handed over keeps
// V' >= V_th for the neurons that spiked in the step before the run (their spikes in
// net->spk), so those are reset first, with the update's own reset arithmetic.
template <bool kSoft>
__global__ __launch_bounds__(256) void k_lif_defer_in(int32_t n, float* V, const uint8_t* spk,
                                                      bs_lif_params p) {
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < n;
       j += (int64_t)gridDim.x * 256)
    if (spk[j]) V[j] = bs_lif_reset<kSoft>(p, V[j]);
}

// ... and after it, each neuron that spiked in the last step gets back its V' of that step:
// the update's membrane step from its V before the step (vprev) and its conductances after
// it, the same operations (bs_lif_vnext) the runner applied before resetting.
template <bool kCuba>
__global__ __launch_bounds__(256) void k_lif_defer_out(int32_t n, float* V, const float* vprev,
                                                       const float* ge, const float* gi,
                                                       const uint8_t* spk, const float* iext,
                                                       const float* istep, bs_lif_params p) {
  if (istep) p.I_ext = *istep;   // the last step's input of a run with per-step inputs
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < n;
       j += (int64_t)gridDim.x * 256) {
    if (!spk[j]) continue;
    bs_lif_params q = p;
    if (iext) q.I_ext = iext[j];
    V[j] = bs_lif_vnext<kCuba>(q, vprev[j], ge[j], gi[j]);
  }
}

template <bool kCuba, bool kSoft>
int lif_run(const bs_net* net, const bs_lif_state* st, const bs_lif_params* p, int64_t t0,
            int32_t steps, int32_t* counts_out, uint32_t* hash_out, uint8_t* raster_out,
            void* workspace, bs_stream_t stream, const char* who, const float* isched) {
  if (!p || !p->deferred_reset || steps <= 0)
    return run<LifModel<kCuba, kSoft>>(net, st, p, t0, steps, counts_out, hash_out, raster_out,
                                       workspace, stream, who, isched);
  int rc = check_net(net, who);
  if (rc) return rc;
  BS_CHECK_ARG(st && workspace, "%s: NULL state/workspace", who);
  NetLayout L;
  if (plan(net, &L)) {
    bs_set_error("%s: n=%d needs more than %d neurons per thread", who, net->n, kMaxNpt);
    return BS_ERR_UNSUPPORTED;
  }
  hipStream_t s = bs_stream(stream);
  const int g = (int)((net->n + 255) / 256 < 2048 ? (net->n + 255) / 256 : 2048);
  k_lif_defer_in<kSoft><<<g, 256, 0, s>>>(net->n, st->V, net->spk, *p);
  BS_CHECK_LAUNCH();
  // all but the last step, then V before it, then the last step
  if (steps > 1) {
    rc = run<LifModel<kCuba, kSoft>>(net, st, p, t0, steps - 1, counts_out, hash_out,
                                     raster_out, workspace, stream, who, isched);
    if (rc) return rc;
  }
  float* vprev = (float*)((char*)workspace + L.off_vprev);
  BS_CHECK_HIP(hipMemcpyAsync(vprev, st->V, (size_t)net->n * sizeof(float),
                              hipMemcpyDeviceToDevice, s));
  const int64_t k = steps - 1;
  rc = run<LifModel<kCuba, kSoft>>(net, st, p, t0 + k, 1, counts_out ? counts_out + k : nullptr,
                                   hash_out ? hash_out + k : nullptr,
                                   raster_out ? raster_out + k * net->n : nullptr, workspace,
                                   stream, who, isched ? isched + k : nullptr);
  if (rc) return rc;
  k_lif_defer_out<kCuba><<<g, 256, 0, s>>>(net->n, st->V, vprev, st->ge, st->gi, net->spk,
                                           net->I_ext, isched ? isched + k : nullptr, *p);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

}  // namespace

namespace {

int lif_run_any(const bs_net* net, const bs_lif_state* st, const bs_lif_params* p, int64_t t0,
                int32_t steps, const float* isched, int32_t* counts_out, uint32_t* hash_out,
                uint8_t* raster_out, void* workspace, bs_stream_t stream, const char* who) {
  if (st) BS_CHECK_ARG(st->V && st->ge && st->gi && st->ref, "%s: NULL state pointer", who);
  if (p) BS_CHECK_ARG(p->inv_tau == p->inv_tau, "%s: inv_tau is NaN", who);
#define BS_RUN(C, S)                                                                    \
  return lif_run<C, S>(net, st, p, t0, steps, counts_out, hash_out, raster_out, workspace,  \
                       stream, who, isched)
  const bool cuba = p && p->cuba, soft = p && p->soft_reset;
  if (cuba) { if (soft) BS_RUN(true, true); else BS_RUN(true, false); }
  if (soft) BS_RUN(false, true);
  BS_RUN(false, false);
#undef BS_RUN
}

int hh_run_any(const bs_net* net, const bs_hh_state* st, const bs_hh_params* p, int64_t t0,
               int32_t steps, const float* isched, int32_t* counts_out, uint32_t* hash_out,
               uint8_t* raster_out, void* workspace, bs_stream_t stream, const char* who) {
  if (st) {
    BS_CHECK_ARG(st->V && st->m && st->h && st->n && st->ge && st->gi,
                 "%s: NULL state pointer", who);
  }
  if (p) BS_CHECK_ARG(p->inv_C == p->inv_C, "%s: inv_C is NaN", who);
  return run<HhModel>(net, st, p, t0, steps, counts_out, hash_out, raster_out, workspace,
                      stream, who, isched);
}

// Checks of the per-step input array of the *_run_inputs entry points.
int check_inputs(const bs_net* net, const float* I_steps, int32_t steps, const char* who) {
  BS_CHECK_ARG(net != nullptr, "%s: net is NULL", who);
  BS_CHECK_ARG(I_steps != nullptr || steps <= 0, "%s: I_steps is NULL", who);
  BS_CHECK_ARG(net->I_ext == nullptr,
               "%s: per-step inputs and per-neuron inputs (net->I_ext) do not combine", who);
  BS_CHECK_ARG(((uintptr_t)I_steps & 3) == 0, "%s: I_steps not 4-byte aligned", who);
  return BS_OK;
}

}  // namespace

extern "C" int bs_coba_lif_run(const bs_net* net, const bs_lif_state* st, const bs_lif_params* p,
                               int64_t t0, int32_t steps, int32_t* counts_out,
                               uint32_t* hash_out, uint8_t* raster_out, void* workspace,
                               bs_stream_t stream) {
  bs_clear_error();
  return lif_run_any(net, st, p, t0, steps, nullptr, counts_out, hash_out, raster_out,
                     workspace, stream, "bs_coba_lif_run");
}

extern "C" int bs_coba_lif_run_inputs(const bs_net* net, const bs_lif_state* st,
                                      const bs_lif_params* p, const float* I_steps, int64_t t0,
                                      int32_t steps, int32_t* counts_out, uint32_t* hash_out,
                                      uint8_t* raster_out, void* workspace,
                                      bs_stream_t stream) {
  bs_clear_error();
  const char* who = "bs_coba_lif_run_inputs";
  int rc = check_inputs(net, I_steps, steps, who);
  if (rc) return rc;
  return lif_run_any(net, st, p, t0, steps, I_steps, counts_out, hash_out, raster_out,
                     workspace, stream, who);
}

extern "C" int bs_coba_hh_run(const bs_net* net, const bs_hh_state* st, const bs_hh_params* p,
                              int64_t t0, int32_t steps, int32_t* counts_out,
                              uint32_t* hash_out, uint8_t* raster_out, void* workspace,
                              bs_stream_t stream) {
  bs_clear_error();
  return hh_run_any(net, st, p, t0, steps, nullptr, counts_out, hash_out, raster_out,
                    workspace, stream, "bs_coba_hh_run");
}

extern "C" int bs_coba_hh_run_inputs(const bs_net* net, const bs_hh_state* st,
                                     const bs_hh_params* p, const float* I_steps, int64_t t0,
                                     int32_t steps, int32_t* counts_out, uint32_t* hash_out,
                                     uint8_t* raster_out, void* workspace, bs_stream_t stream) {
  bs_clear_error();
  const char* who = "bs_coba_hh_run_inputs";
  int rc = check_inputs(net, I_steps, steps, who);
  if (rc) return rc;
  return hh_run_any(net, st, p, t0, steps, I_steps, counts_out, hash_out, raster_out,
                    workspace, stream, who);
}

extern "C" int bs_net_error(const void* workspace, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(workspace != nullptr, "bs_net_error: workspace is NULL");
  uint32_t e = 0;
  BS_CHECK_HIP(hipMemcpyAsync(&e, workspace, sizeof(e), hipMemcpyDeviceToHost,
                              bs_stream(stream)));
  BS_CHECK_HIP(hipStreamSynchronize(bs_stream(stream)));
  if (e == 2u) {
    bs_set_error("runner: a per-synapse weight is not finite (or too large for the fixed-point "
                 "input sums)");
    return -2;
  }
  if (e) bs_set_error("runner: a wait for a count word hit its spin limit");
  return e ? -1 : 0;
}

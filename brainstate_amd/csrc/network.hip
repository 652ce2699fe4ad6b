// Whole-loop runners for E/I networks: one persistent (cooperative) launch runs T steps.
//
// Why persistent: one step of the 1M-neuron COBA net moves ~34 MB, ~4 us at 8 TB/s,
// which is the same order as a kernel launch.  A per-step chain of launches (update,
// compaction, two scatters) would be launch-bound.  Here each workgroup owns a fixed
// slice of neurons for the whole run and keeps their state in registers; per step it
//   1. reads (and clears) its neurons' pending inputs acc[cur][E|I][j],
//   2. runs the fused Expon + COBA + neuron update,
//   3. compacts its spikes into an ordered LDS list (wave ballot + mbcnt rank),
//   4. scatters the synapse rows of its own spiking neurons into acc[nxt] with hardware
//      fp32 atomics (rows are contiguous: 64 lanes read 256 B of indices per chunk),
//   5. meets the other workgroups at one grid barrier.
// Steps 1-4 need no barrier between them because a workgroup only scatters spikes it
// produced itself, and acc is double-buffered: nobody writes acc[cur] during step t.
#include "neuron_dev.h"

namespace {

constexpr int kBlock = 1024;
constexpr int kWaves = kBlock / BS_WAVE;

struct bs_grid_bar {
  uint32_t count;
  uint32_t pad0[31];
  uint32_t gen;
  uint32_t pad1[31];
};

struct NetArgs {
  int32_t n, n_exc, k_e, k_i;
  const int32_t* idx_e;
  const float* w_e;
  float w_e_homo;
  const int32_t* idx_i;
  const float* w_i;
  float w_i_homo;
  float* acc;
  uint8_t* spk;
  int32_t steps, phase;
  int32_t* counts;
  uint32_t* hash;
  uint8_t* raster;
  bs_grid_bar* bar;
};

// Sense-free generation barrier over all workgroups of a co-resident grid.  Every
// workgroup arrives exactly once per call, so every wait ends.
__device__ __forceinline__ void grid_barrier(bs_grid_bar* bar, uint32_t nblocks, uint32_t& gen) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t g = gen;
    const uint32_t arrived =
        __hip_atomic_fetch_add(&bar->count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived == nblocks - 1) {
      __hip_atomic_store(&bar->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&bar->gen, g + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      while (__hip_atomic_load(&bar->gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == g)
        __builtin_amdgcn_s_sleep(1);
    }
  }
  gen = gen + 1u;
  __syncthreads();
}

// ---- neuron models: register-resident state, one fused update per neuron-step ----

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
  __device__ static bool update(const Params& p, Regs& r, float in_e, float in_i) {
    return bs_lif_update(p, r.V, r.ge, r.gi, r.ref, in_e, in_i);
  }
};

struct HhModel {
  using Params = bs_hh_params;
  using State = bs_hh_state;
  struct Regs {
    float V, m, h, n, ge, gi;
  };
  __device__ static Regs load(const State& s, int64_t j) {
    return Regs{s.V[j], s.m[j], s.h[j], s.n[j], s.ge[j], s.gi[j]};
  }
  __device__ static void store(const State& s, int64_t j, const Regs& r) {
    s.V[j] = r.V;
    s.m[j] = r.m;
    s.h[j] = r.h;
    s.n[j] = r.n;
    s.ge[j] = r.ge;
    s.gi[j] = r.gi;
  }
  __device__ static bool update(const Params& p, Regs& r, float in_e, float in_i) {
    return bs_hh_update(p, r.V, r.m, r.h, r.n, r.ge, r.gi, in_e, in_i);
  }
};

template <class Model, int NPT, bool kHet>
__global__ __launch_bounds__(kBlock) void k_run(NetArgs a, typename Model::State st,
                                                typename Model::Params p) {
  __shared__ int32_t s_list[NPT * kBlock];
  __shared__ int32_t s_wave[kWaves];
  __shared__ uint32_t s_hash;

  const int lane = bs_lane();
  const int wid = threadIdx.x / BS_WAVE;
  const uint32_t nblocks = gridDim.x;
  const int64_t base = (int64_t)blockIdx.x * (NPT * kBlock);
  const int64_t n = a.n;
  uint32_t gen = 0;
  if (threadIdx.x == 0)
    gen = __hip_atomic_load(&a.bar->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  typename Model::Regs r[NPT];
#pragma unroll
  for (int q = 0; q < NPT; ++q) {
    const int64_t j = base + q * kBlock + threadIdx.x;
    if (j < n) r[q] = Model::load(st, j);
  }
  bool last[NPT];
#pragma unroll
  for (int q = 0; q < NPT; ++q) last[q] = false;

  const int32_t cpr_e = (a.k_e + BS_WAVE - 1) / BS_WAVE;
  const int32_t cpr_i = (a.k_i + BS_WAVE - 1) / BS_WAVE;
  const int32_t cpr = cpr_e > cpr_i ? cpr_e : cpr_i;

  for (int32_t t = 0; t < a.steps; ++t) {
    const int cur = (a.phase + t) & 1;
    float* acc_cur = a.acc + (int64_t)cur * 2 * n;
    float* acc_nxt = a.acc + (int64_t)(cur ^ 1) * 2 * n;

    // 1-2: inputs + fused update
    float in_e[NPT], in_i[NPT];
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int64_t j = base + q * kBlock + threadIdx.x;
      in_e[q] = 0.0f;
      in_i[q] = 0.0f;
      if (j < n) {
        in_e[q] = acc_cur[j];
        in_i[q] = acc_cur[n + j];
      }
    }
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int64_t j = base + q * kBlock + threadIdx.x;
      if (j < n) {
        acc_cur[j] = 0.0f;
        acc_cur[n + j] = 0.0f;
        last[q] = Model::update(p, r[q], in_e[q], in_i[q]);
      }
    }

    // 3: ordered compaction of this workgroup's spikes into LDS
    int32_t count = 0;
    uint32_t h = 0;
    if (threadIdx.x == 0) s_hash = 0;
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int64_t j = base + q * kBlock + threadIdx.x;
      const bool s = last[q];
      const uint64_t m = bs_ballot(s);
      if (lane == 0) s_wave[wid] = __popcll(m);
      __syncthreads();
      int32_t off = count, tot = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int32_t c = s_wave[w];
        off += (w < wid) ? c : 0;
        tot += c;
      }
      if (s) {
        s_list[off + bs_rank_below(m)] = (int32_t)j;
        h += bs_mix32((uint32_t)j);
      }
      if (a.raster && j < n) a.raster[(int64_t)t * n + j] = s ? 1 : 0;
      count += tot;
      __syncthreads();
    }
    if (a.hash && h) atomicAdd(&s_hash, h);

    // 4: scatter this workgroup's spikes (E rows for j < n_exc, I rows otherwise)
    const int32_t items = count * cpr;
    for (int32_t it = wid; it < items; it += kWaves) {
      const int32_t ai = it / cpr;
      const int32_t c = it - ai * cpr;
      const int32_t i = s_list[ai];
      const bool exc = i < a.n_exc;
      const int32_t k = exc ? a.k_e : a.k_i;
      const int32_t tt = c * BS_WAVE + lane;
      if (tt < k) {
        const int64_t s = (int64_t)(exc ? i : i - a.n_exc) * k + tt;
        const int32_t tgt = exc ? a.idx_e[s] : a.idx_i[s];
        float v;
        if (kHet) v = exc ? a.w_e[s] : a.w_i[s];
        else v = exc ? a.w_e_homo : a.w_i_homo;
        if ((uint32_t)tgt < (uint32_t)n)
          bs_atomic_add_f32(acc_nxt + (exc ? 0 : n) + tgt, v);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      if (a.counts && count) atomicAdd(&a.counts[t], count);
      if (a.hash && s_hash) atomicAdd(&a.hash[t], s_hash);
    }

    // 5: all inputs for step t+1 are in acc[nxt]
    grid_barrier(a.bar, nblocks, gen);
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

__global__ void k_zero_u32(uint32_t* p, int32_t n) {
  for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p[i] = 0u;
}

template <class Model, int NPT, bool kHet>
int occupancy() {
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_run<Model, NPT, kHet>, kBlock, 0) !=
      hipSuccess)
    return 0;
  return nb;
}

int pick_blocks_per_cu(const bs_net* net) {
  return net->blocks_per_cu > 0 ? net->blocks_per_cu : 1;
}

int npt_for(int64_t n, int64_t threads) {
  const int64_t need = (n + threads - 1) / threads;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  if (need <= 16) return 16;
  return -1;
}

template <class Model, int NPT, bool kHet>
int launch_one(const NetArgs& a, const typename Model::State& st, const typename Model::Params& p,
               int grid, hipStream_t s) {
  const int occ = occupancy<Model, NPT, kHet>();
  if (occ * bs_num_cus() < grid) {
    bs_set_error("runner: grid of %d workgroups cannot be co-resident (occupancy %d x %d CUs)",
                 grid, occ, bs_num_cus());
    return BS_ERR_UNSUPPORTED;
  }
  NetArgs aa = a;
  typename Model::State ss = st;
  typename Model::Params pp = p;
  void* args[] = {(void*)&aa, (void*)&ss, (void*)&pp};
  BS_CHECK_HIP(hipLaunchCooperativeKernel((const void*)k_run<Model, NPT, kHet>, dim3(grid),
                                          dim3(kBlock), args, 0, s));
  return BS_OK;
}

template <class Model, bool kHet>
int dispatch_npt(int npt, const NetArgs& a, const typename Model::State& st,
                 const typename Model::Params& p, int grid, hipStream_t s) {
  switch (npt) {
    case 1: return launch_one<Model, 1, kHet>(a, st, p, grid, s);
    case 2: return launch_one<Model, 2, kHet>(a, st, p, grid, s);
    case 4: return launch_one<Model, 4, kHet>(a, st, p, grid, s);
    case 8: return launch_one<Model, 8, kHet>(a, st, p, grid, s);
    case 16: return launch_one<Model, 16, kHet>(a, st, p, grid, s);
  }
  bs_set_error("runner: unsupported neurons-per-thread %d", npt);
  return BS_ERR_UNSUPPORTED;
}

int check_net(const bs_net* net, const char* who) {
  BS_CHECK_ARG(net != nullptr, "%s: net is NULL", who);
  BS_CHECK_ARG(net->n > 0 && net->n_exc >= 0 && net->n_exc <= net->n,
               "%s: bad sizes n=%d n_exc=%d", who, net->n, net->n_exc);
  BS_CHECK_ARG(net->k_e >= 0 && net->k_i >= 0, "%s: negative fan-out", who);
  BS_CHECK_ARG(net->acc && net->spk, "%s: acc/spk is NULL", who);
  BS_CHECK_ARG(net->n_exc == 0 || net->k_e == 0 || net->idx_e, "%s: idx_e is NULL", who);
  BS_CHECK_ARG(net->n_exc == net->n || net->k_i == 0 || net->idx_i, "%s: idx_i is NULL", who);
  BS_CHECK_ARG((net->w_e == nullptr) == (net->w_i == nullptr),
               "%s: w_e and w_i must both be given or both be NULL", who);
  return BS_OK;
}

template <class Model>
int run(const bs_net* net, const typename Model::State* st, const typename Model::Params* p,
        int32_t steps, int32_t phase, int32_t* counts_out, uint32_t* hash_out,
        uint8_t* raster_out, void* workspace, bs_stream_t stream, const char* who) {
  bs_clear_error();
  int rc = check_net(net, who);
  if (rc) return rc;
  BS_CHECK_ARG(st && p && workspace, "%s: NULL state/params/workspace", who);
  BS_CHECK_ARG(steps >= 0, "%s: steps=%d < 0", who, steps);
  BS_CHECK_ARG(phase == 0 || phase == 1, "%s: phase must be 0 or 1", who);
  if (steps == 0) return BS_OK;
  const int grid = bs_net_grid_blocks(net);
  BS_CHECK_ARG(grid > 0, "%s: %s", who, bs_last_error());
  const int npt = npt_for(net->n, (int64_t)grid * kBlock);
  if (npt < 0) {
    bs_set_error("%s: n=%d exceeds 16 neurons per thread on %d workgroups", who, net->n, grid);
    return BS_ERR_UNSUPPORTED;
  }
  hipStream_t s = bs_stream(stream);
  if (counts_out) {
    k_zero_u32<<<(steps + 255) / 256, 256, 0, s>>>((uint32_t*)counts_out, steps);
    BS_CHECK_LAUNCH();
  }
  if (hash_out) {
    k_zero_u32<<<(steps + 255) / 256, 256, 0, s>>>(hash_out, steps);
    BS_CHECK_LAUNCH();
  }
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
  a.acc = net->acc;
  a.spk = net->spk;
  a.steps = steps;
  a.phase = phase;
  a.counts = counts_out;
  a.hash = hash_out;
  a.raster = raster_out;
  a.bar = (bs_grid_bar*)workspace;
  if (net->w_e != nullptr) return dispatch_npt<Model, true>(npt, a, *st, *p, grid, s);
  return dispatch_npt<Model, false>(npt, a, *st, *p, grid, s);
}

}  // namespace

extern "C" size_t bs_net_workspace_size(void) { return sizeof(bs_grid_bar); }

extern "C" int bs_net_grid_blocks(const bs_net* net) {
  if (net == nullptr) {
    bs_set_error("bs_net_grid_blocks: net is NULL");
    return -1;
  }
  const int cus = bs_num_cus();
  int bpc = pick_blocks_per_cu(net);
  // never more workgroups than neurons need
  const int64_t need = ((int64_t)net->n + kBlock - 1) / kBlock;
  int64_t grid = (int64_t)bpc * cus;
  if (grid > need) grid = need;
  if (grid < 1) grid = 1;
  return (int)grid;
}

extern "C" int bs_coba_lif_run(const bs_net* net, const bs_lif_state* st, const bs_lif_params* p,
                               int32_t steps, int32_t phase, int32_t* counts_out,
                               uint32_t* hash_out, uint8_t* raster_out, void* workspace,
                               bs_stream_t stream) {
  if (st) {
    BS_CHECK_ARG(st->V && st->ge && st->gi && st->ref, "bs_coba_lif_run: NULL state pointer");
  }
  if (p) BS_CHECK_ARG(p->tau != 0.0f, "bs_coba_lif_run: tau must be nonzero");
  return run<LifModel>(net, st, p, steps, phase, counts_out, hash_out, raster_out, workspace,
                       stream, "bs_coba_lif_run");
}

extern "C" int bs_coba_hh_run(const bs_net* net, const bs_hh_state* st, const bs_hh_params* p,
                              int32_t steps, int32_t phase, int32_t* counts_out,
                              uint32_t* hash_out, uint8_t* raster_out, void* workspace,
                              bs_stream_t stream) {
  if (st) {
    BS_CHECK_ARG(st->V && st->m && st->h && st->n && st->ge && st->gi,
                 "bs_coba_hh_run: NULL state pointer");
  }
  if (p) BS_CHECK_ARG(p->C != 0.0f, "bs_coba_hh_run: C must be nonzero");
  return run<HhModel>(net, st, p, steps, phase, counts_out, hash_out, raster_out, workspace,
                      stream, "bs_coba_hh_run");
}

// N1: spike compaction.  bool/float spike vector -> ascending active-index list + count.
//
// One pass.  Each workgroup takes a ticket (its tile number), ballots its tile one
// 256-element sweep at a time (wave ballot + mbcnt rank, per-wave totals in LDS) into
// an ordered LDS list, then finds its global offset by decoupled look-back over the
// tiles with smaller tickets and writes the list out coalesced.
#include "common.h"

#include <mutex>

namespace {

constexpr int kBlock = 256;
constexpr int kSweeps = 16;
constexpr int kTile = kBlock * kSweeps;   // 4096 spikes per workgroup
constexpr int kWaves = kBlock / BS_WAVE;

__device__ __forceinline__ bool is_event(const uint8_t* p, int64_t i) { return p[i] != 0; }
__device__ __forceinline__ bool is_event(const float* p, int64_t i) { return p[i] != 0.0f; }

__device__ __forceinline__ uint64_t pack_status(uint32_t epoch, uint32_t flag, uint32_t v) {
  return ((uint64_t)(epoch + 1u) << 32) | ((uint64_t)flag << 30) | (uint64_t)(v & 0x3FFFFFFFu);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_compact(const T* __restrict__ spk, int32_t n,
                                                    int32_t* __restrict__ idx_out,
                                                    int32_t* __restrict__ count_out,
                                                    bs_scan_ws* __restrict__ ws,
                                                    uint32_t nblocks) {
  __shared__ int32_t s_list[kTile];
  __shared__ int32_t s_wave[kWaves];
  __shared__ uint32_t s_ticket, s_epoch;
  __shared__ int32_t s_excl;

  if (threadIdx.x == 0) {
    s_ticket = atomicAdd(&ws->ticket, 1u);
    s_epoch = __hip_atomic_load(&ws->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const uint32_t tile = s_ticket;
  const uint32_t epoch = s_epoch;
  const int lane = bs_lane();
  const int wid = threadIdx.x / BS_WAVE;

  int32_t count = 0;  // uniform across the workgroup
  const int64_t base = (int64_t)tile * kTile;
  for (int s = 0; s < kSweeps; ++s) {
    const int64_t e = base + s * kBlock + threadIdx.x;
    const bool p = e < n && is_event(spk, e);
    const uint64_t m = bs_ballot(p);
    if (lane == 0) s_wave[wid] = __popcll(m);
    __syncthreads();
    int32_t off = count, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int32_t c = s_wave[w];
      off += (w < wid) ? c : 0;
      tot += c;
    }
    if (p) s_list[off + bs_rank_below(m)] = (int32_t)e;
    count += tot;
    __syncthreads();
  }

  if (threadIdx.x == 0) {
    uint64_t* st = bs_scan_status(ws);
    int32_t excl = 0;
    if (tile == 0) {
      __hip_atomic_store(&st[0], pack_status(epoch, BS_ST_INC, count), __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __hip_atomic_store(&st[tile], pack_status(epoch, BS_ST_AGG, count), __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_AGENT);
      int64_t j = (int64_t)tile - 1;
      while (true) {
        const uint64_t v = __hip_atomic_load(&st[j], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)(v >> 32) != epoch + 1u) {  // tile j has not published yet
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        excl += (int32_t)(v & 0x3FFFFFFFu);
        if (((v >> 30) & 3u) == BS_ST_INC) break;
        --j;
      }
      __hip_atomic_store(&st[tile], pack_status(epoch, BS_ST_INC, excl + count),
                         __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_excl = excl;
    if (tile == nblocks - 1) *count_out = excl + count;
  }
  __syncthreads();
  const int32_t excl = s_excl;
  for (int32_t i = threadIdx.x; i < count; i += kBlock) idx_out[excl + i] = s_list[i];

  if (threadIdx.x == 0) {
    // The last workgroup to finish resets the tickets and opens a new epoch.
    const uint32_t d = __hip_atomic_fetch_add(&ws->done, 1u, __ATOMIC_ACQ_REL,
                                              __HIP_MEMORY_SCOPE_AGENT);
    if (d == nblocks - 1) {
      __hip_atomic_store(&ws->ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ws->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ws->epoch, epoch + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

__global__ void k_set_i32(int32_t* p, int32_t v) { *p = v; }

__global__ void k_zero_u64(uint64_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0ull;
}

// ---- bs_spike_compact_noalloc: the scan workspace in a file-scope device array ----
// The scan header and one status word per 4096-spike tile, for up to kNoAllocTiles tiles.
// Each device holds its own copy; host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device (the array's name is a host-side
// stand-in, not a device address).
constexpr int64_t kNoAllocTiles = 16384;  // n <= 16384 * 4096 = 67,108,864 spikes
constexpr size_t kScratchBytes = BS_SCAN_WS_HEADER + (size_t)kNoAllocTiles * sizeof(uint64_t);
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];  // device address of `scratch`, per device (null: not yet)

// Device address of this device's scratch.  The first call on a device looks it up with that
// device current and clears it with a kernel on `s` (the scan counters must start at zero;
// every later call leaves them at rest again).
int scratch_for_current_device(hipStream_t s, void** out) {
  int dev = -1;
  BS_CHECK_HIP(hipGetDevice(&dev));
  BS_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "bs_spike_compact_noalloc: device %d beyond %d",
               dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    BS_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    BS_CHECK_ARG(p != nullptr, "bs_spike_compact_noalloc: no device address for the scratch");
    k_zero_u64<<<64, 256, 0, s>>>((uint64_t*)p, (int64_t)(kScratchBytes / sizeof(uint64_t)));
    BS_CHECK_LAUNCH();
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return BS_OK;
}

}  // namespace

extern "C" size_t bs_spike_compact_workspace_size(int32_t n) {
  const int64_t nb = n > 0 ? ((int64_t)n + kTile - 1) / kTile : 0;
  return BS_SCAN_WS_HEADER + (size_t)nb * sizeof(uint64_t);
}

extern "C" int bs_spike_compact(const void* spk, int32_t spk_dtype, int32_t n, int32_t* idx_out,
                                int32_t* count_out, void* workspace, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n >= 0 && n < (1 << 30), "bs_spike_compact: n=%d out of range [0, 2^30)", n);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_spike_compact: unknown spike dtype %d", spk_dtype);
  BS_CHECK_ARG(count_out != nullptr, "bs_spike_compact: count_out is NULL");
  hipStream_t s = bs_stream(stream);
  if (n == 0) {
    k_set_i32<<<1, 1, 0, s>>>(count_out, 0);
    BS_CHECK_LAUNCH();
    return BS_OK;
  }
  BS_CHECK_ARG(spk && idx_out && workspace, "bs_spike_compact: NULL pointer");
  const uint32_t nb = (uint32_t)(((int64_t)n + kTile - 1) / kTile);
  bs_scan_ws* ws = (bs_scan_ws*)workspace;
  if (spk_dtype == BS_SPK_U8)
    k_compact<uint8_t><<<nb, kBlock, 0, s>>>((const uint8_t*)spk, n, idx_out, count_out, ws, nb);
  else
    k_compact<float><<<nb, kBlock, 0, s>>>((const float*)spk, n, idx_out, count_out, ws, nb);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_spike_compact_noalloc(const void* spk, int32_t spk_dtype, int32_t n,
                                        int32_t* idx_out, int32_t* count_out,
                                        bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n >= 0 && n <= kNoAllocTiles * kTile,
               "bs_spike_compact_noalloc: n=%d exceeds the maximum %lld (a static scratch of "
               "%zu bytes per device); use bs_spike_compact with a workspace",
               n, (long long)(kNoAllocTiles * kTile), kScratchBytes);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_spike_compact_noalloc: unknown spike dtype %d", spk_dtype);
  BS_CHECK_ARG(count_out != nullptr, "bs_spike_compact_noalloc: count_out is NULL");
  hipStream_t s = bs_stream(stream);
  if (n == 0) {
    k_set_i32<<<1, 1, 0, s>>>(count_out, 0);
    BS_CHECK_LAUNCH();
    return BS_OK;
  }
  BS_CHECK_ARG(spk && idx_out, "bs_spike_compact_noalloc: NULL pointer");
  void* ws = nullptr;
  const int rc = scratch_for_current_device(s, &ws);
  if (rc) return rc;
  const uint32_t nb = (uint32_t)(((int64_t)n + kTile - 1) / kTile);
  if (spk_dtype == BS_SPK_U8)
    k_compact<uint8_t><<<nb, kBlock, 0, s>>>((const uint8_t*)spk, n, idx_out, count_out,
                                             (bs_scan_ws*)ws, nb);
  else
    k_compact<float><<<nb, kBlock, 0, s>>>((const float*)spk, n, idx_out, count_out,
                                           (bs_scan_ws*)ws, nb);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

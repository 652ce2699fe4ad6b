// N1: spike compaction.  bool/float spike vector -> ascending active-index list + count.
//
// One pass.  Each workgroup takes a ticket (its tile number), loads its tile at once (64
// consecutive spikes per thread), places each thread's active spikes by a wave prefix of the
// per-thread counts and one round of per-wave totals in LDS, then finds its global offset by
// decoupled look-back over the tiles with smaller tickets and writes its indices out.
#include "common.h"

#include <mutex>

namespace {

constexpr int kBlock = 256;
constexpr int kPerThread = 64;  // consecutive spikes per thread
constexpr int kTile = kBlock * kPerThread;   // 16384 spikes per workgroup
constexpr int kWaves = kBlock / BS_WAVE;

__device__ __forceinline__ bool is_event(const uint8_t* p, int64_t i) { return p[i] != 0; }
__device__ __forceinline__ bool is_event(const float* p, int64_t i) { return p[i] != 0.0f; }

// Status word: tag epoch + 1 (never 0, the value of a cleared word: the epoch stays in
// [0, 2^32 - 2]), 2 flag bits, a 30-bit count.
__device__ __forceinline__ uint64_t pack_status(uint32_t epoch, uint32_t flag, uint32_t v) {
  return ((uint64_t)(epoch + 1u) << 32) | ((uint64_t)flag << 30) | (uint64_t)(v & 0x3FFFFFFFu);
}

// The epoch after `e`, skipping 2^32 - 1 so that no tag is 0.  A tag comes back after
// 2^32 - 1 calls on one workspace; a status word left from that long ago (a tile no call in
// between reached) would read as published, which needs 2^32 - 1 calls of fewer tiles first.
__device__ __forceinline__ uint32_t next_epoch(uint32_t e) {
  return e >= 0xFFFFFFFEu ? 0u : e + 1u;
}

// 16 consecutive spikes of thread t as bit u = spike base + 16 t + u (kVec: one 16-byte load
// of bytes, or four of floats, from a 16-byte aligned tile that lies wholly inside [0, n)).
template <typename T, bool kVec>
__device__ __forceinline__ uint32_t spike_bits16(const T* __restrict__ spk, int32_t n,
                                                 int64_t e0) {
  uint32_t m = 0;
  if (kVec && e0 + 16 <= n) {
    if constexpr (sizeof(T) == 1) {
      const uint4 x = *(const uint4*)(spk + e0);
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // bit 7 of each nonzero byte, gathered into bits 21..24 by one multiply
        const uint32_t hi = ((((w[q] & 0x7f7f7f7fu) + 0x7f7f7f7fu) | w[q]) & 0x80808080u) >> 7;
        m |= ((hi * 0x00204081u) >> 21 & 0xFu) << (4 * q);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 x = *(const float4*)(spk + e0 + 4 * q);
        m |= (x.x != 0.0f ? 1u : 0u) << (4 * q) | (x.y != 0.0f ? 2u : 0u) << (4 * q) |
             (x.z != 0.0f ? 4u : 0u) << (4 * q) | (x.w != 0.0f ? 8u : 0u) << (4 * q);
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (e0 + u < n && is_event(spk, e0 + u)) m |= 1u << u;
  }
  return m;
}

// One tile of kTile spikes per workgroup: thread t loads spikes 16 t .. 16 t + 15 of the tile
// together (one memory round trip for the whole tile), counts them, and a workgroup prefix of
// the counts gives each thread its place in the tile's ascending list.
template <typename T, bool kVec>
__global__ __launch_bounds__(kBlock) void k_compact(const T* __restrict__ spk, int32_t n,
                                                    int32_t* __restrict__ idx_out,
                                                    int32_t* __restrict__ count_out,
                                                    bs_scan_ws* __restrict__ ws,
                                                    uint32_t nblocks) {
  static_assert(kPerThread % 16 == 0 && kPerThread <= 64, "whole 16-spike loads, 64-bit mask");
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

  const int64_t base = (int64_t)tile * kTile;
  const int64_t e0 = base + kPerThread * (int64_t)threadIdx.x;
  uint64_t bits = 0;
#pragma unroll
  for (int q = 0; q < kPerThread / 16; ++q)
    bits |= (uint64_t)spike_bits16<T, kVec>(spk, n, e0 + 16 * q) << (16 * q);
  // inclusive prefix of the per-thread counts within the wave, then across the waves
  const int32_t c = __popcll(bits);
  int32_t inc = c;
#pragma unroll
  for (int o = 1; o < BS_WAVE; o <<= 1) {
    const int32_t v = __shfl_up(inc, o);
    if (lane >= o) inc += v;
  }
  if (lane == BS_WAVE - 1) s_wave[wid] = inc;
  __syncthreads();
  int32_t off = inc - c, count = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int32_t t = s_wave[w];
    off += (w < wid) ? t : 0;
    count += t;
  }

  // Status words carry their own value (epoch, flag and count in one 64-bit word), and no
  // workgroup reads another's list, so relaxed device-scope atomics are all the look-back
  // needs: no release / acquire, each of which costs an L2 write-back or invalidate here
  // (with them every tile waited ~0.3 us on its predecessor: 61 us for 1M spikes).  The
  // last tile's reset of the ticket and the epoch is read by the next launch only.
  // The look-back is wave-wide: wave 0 reads the statuses of the 64 nearest tiles not yet
  // added in one round trip (lane l: tile j - l), adds the published ones up to the nearest
  // inclusive prefix, and goes on from the first unpublished one (at 4M spikes the one-status
  // walk took 35 us, most of it round trips over tiles that had published only their count).
  if (wid == 0) {
    uint64_t* st = bs_scan_status(ws);
    int32_t excl = 0;
    if (tile == 0) {
      if (lane == 0)
        __hip_atomic_store(&st[0], pack_status(epoch, BS_ST_INC, count), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else {
      if (lane == 0)
        __hip_atomic_store(&st[tile], pack_status(epoch, BS_ST_AGG, count), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      int64_t j = (int64_t)tile - 1;  // the newest tile not yet added (wave-uniform)
      while (true) {
        const int64_t jj = j - lane;
        const uint64_t v = jj >= 0 ? __hip_atomic_load(&st[jj], __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : pack_status(epoch, BS_ST_INC, 0);  // before tile 0
        const bool pub = (uint32_t)(v >> 32) == epoch + 1u;
        const uint64_t m_unpub = bs_ballot(!pub);
        const uint64_t m_inc = bs_ballot(pub && ((v >> 30) & 3u) == BS_ST_INC);
        const int f_unpub = m_unpub ? (int)__builtin_ctzll(m_unpub) : BS_WAVE;
        const int f_inc = m_inc ? (int)__builtin_ctzll(m_inc) : BS_WAVE;
        // lanes [0, take) are published: up to and including the nearest inclusive prefix
        const int take = f_inc < f_unpub ? f_inc + 1 : f_unpub;
        int32_t val = lane < take ? (int32_t)(v & 0x3FFFFFFFu) : 0;
#pragma unroll
        for (int o = BS_WAVE / 2; o > 0; o >>= 1) val += __shfl_xor(val, o);
        excl += val;
        if (f_inc < f_unpub) break;
        j -= take;
        if (take == 0) __builtin_amdgcn_s_sleep(1);  // the newest one has not published yet
      }
      if (lane == 0)
        __hip_atomic_store(&st[tile], pack_status(epoch, BS_ST_INC, excl + count),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) {
      s_excl = excl;
      if (tile == nblocks - 1) *count_out = excl + count;
    }
  }
  __syncthreads();
  int32_t pos = s_excl + off;
  for (uint64_t m = bits; m; m &= m - 1) idx_out[pos++] = (int32_t)(e0 + __builtin_ctzll(m));

  if (threadIdx.x == 0 && tile == nblocks - 1) {
    // The last tile resets the ticket and opens a new epoch: its look-back ended on an
    // inclusive prefix, so every tile has taken its ticket and read the epoch (a counter of
    // finished workgroups for this, like the ticket one atomic on one word per workgroup,
    // serialised at ~7 ns each: 29.5 -> 22.7 us for 4M spikes without it).  Tickets (not the
    // block index) order the tiles, so a tile waits only on tiles that have started.
    __hip_atomic_store(&ws->ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ws->epoch, next_epoch(epoch), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ void k_set_i32(int32_t* p, int32_t v) { *p = v; }

void launch_compact(const void* spk, int32_t spk_dtype, int32_t n, int32_t* idx_out,
                    int32_t* count_out, bs_scan_ws* ws, uint32_t nb, hipStream_t s) {
  const bool vec = ((uintptr_t)spk & 15) == 0;  // tiles start at multiples of 16 elements
#define BS_CP(T, V) \
  k_compact<T, V><<<nb, kBlock, 0, s>>>((const T*)spk, n, idx_out, count_out, ws, nb)
  if (spk_dtype == BS_SPK_U8) { if (vec) BS_CP(uint8_t, true); else BS_CP(uint8_t, false); }
  else { if (vec) BS_CP(float, true); else BS_CP(float, false); }
#undef BS_CP
}

__global__ void k_zero_u64(uint64_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0ull;
}

// ---- bs_spike_compact_noalloc: the scan workspace in a file-scope device array ----
// The scan header and one status word per 16384-spike tile, for up to kNoAllocTiles tiles.
// Each device holds its own copy; host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device (the array's name is a host-side
// stand-in, not a device address).
constexpr int64_t kNoAllocTiles = 4096;  // n <= 4096 * 16384 = 67,108,864 spikes
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
  launch_compact(spk, spk_dtype, n, idx_out, count_out, ws, nb, s);
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
  launch_compact(spk, spk_dtype, n, idx_out, count_out, (bs_scan_ws*)ws, nb, s);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

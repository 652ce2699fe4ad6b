// N2c: batched event x dense weight (EventLinear).
//
// out[b, j] = sum of W[i, j] over the inputs i with spk[b, i] != 0 (or spk[b, i] * W[i, j]).
// For 64 x 4096 spikes at 5 % and a 4096 x 4096 fp32 W about 3,940 of the 4,096 rows
// of W are selected by at least one batch row, so every step reads almost all of W (64 MiB),
// while the (batch row, active input) pairs number ~13,100: a kernel that fetches a W row
// segment once per pair moves ~210 MB from L2, one that fetches it once per step 64 MiB.
//
// Tiling: a workgroup owns 64*V output columns (lane = V consecutive columns) of 64 batch
// rows (16 waves, 4 batch rows each) over one chunk of consecutive input rows.  It stages W
// through LDS in blocks of 64 rows, prefetched kDepth blocks ahead in registers, so each
// element of W is fetched once per step and shared by all 64 batch rows.  For each block a
// wave turns the spikes of its 4 batch rows into LDS lists of active rows (one ballot and
// one LDS write per row: lane l holds input l of the block; an active lane writes its row's
// byte offset at its rank, inactive lanes write padding that points at a zero row), reads
// the first 8 entries back before the barrier, and after it issues all its W reads at once
// and adds in ascending input order (the padding adds +0.0, which leaves every sum as is).
// Cost model from the hardware counters: the kernel is bound by VALU issue (~160 VALU per
// wave per block, most of it per-(batch row, block) list work rather than per event).
//
// Chunks: bs_event_dense_chunks() splits the inputs into S chunks of L rows so that the grid
// fills the chip (about 256 workgroups) when the output is narrow.  Each chunk's sum is
// formed in ascending input order from 0; with S > 1 every workgroup stores its partial
// sums with device-scope stores, waits for them to complete, and takes a ticket on its
// (column tile, batch group) counter; the workgroup that draws the last ticket adds the S
// partials in chunk order, ((P_0 + P_1) + P_2) + ..., and writes out (device-scope loads:
// no cache writeback or invalidate is needed).  It also clears the counter, so the
// workspace stays ready for the next call.  The order depends only on (batch, n_in, n_out),
// so results are reproducible run to run and device to device.
//
// XCD-aware placement: workgroups are dispatched to the 8 XCDs round-robin; logical
// workgroups are renumbered so that consecutive ones (the column tiles of one chunk, which
// read the same spike bytes) share an XCD and its L2.
#include "bs_math.h"
#include "common.h"

namespace {

constexpr int kBlock = 256;   // reverse-mode kernels
constexpr int kXcds = 8;      // MI355X: 8 XCDs, each with its own L2

constexpr int kDB = 1024;                 // forward: threads per workgroup
constexpr int kDWaves = kDB / BS_WAVE;    // 16
constexpr int kGroupRows = 64;            // batch rows per workgroup
constexpr int kRowsPerWave = kGroupRows / kDWaves;  // 4
constexpr int kBlk = 64;                  // input rows per LDS block (one ballot)
constexpr int kList = kBlk + 12;          // list entries per (wave, batch row): 64 + padding
constexpr int kDump = kList - 1;          // slot written by lanes with nothing to record
// Measured on MI355X for 64 x 4096 spikes at 5 % and W 4096^2: V = 2 with 8 chunks 28 us,
// V = 1 with 4 chunks 30 us, V = 4 120 us (LDS of 152 KiB per workgroup and 64 KiB partials);
// a 256-workgroup launch alone costs ~4.3 us.
constexpr int kV = 2;                     // output columns per lane (workgroup: 64 * V)
constexpr int kTileCols = BS_WAVE * kV;
constexpr int kTargetGroups = 256;        // workgroups the chunk plan aims for
constexpr int kDepth = 2;                 // W blocks in flight per thread (registers)
constexpr int kMaxChunks = 8;             // chunk partials the last workgroup adds

// Spike byte/float -> event flag (any nonzero value is an event).
__device__ __forceinline__ bool nz(uint8_t x) { return x != 0; }
__device__ __forceinline__ bool nz(float x) { return x != 0.0f; }

struct DensePlan {
  int32_t tiles;       // column tiles of 64 * V
  int32_t groups;      // batch groups of 64
  int32_t chunks;      // S
  int32_t chunk_rows;  // L (a multiple of 64)
};

// Chunk plan: a function of the shape only (never of the device), so the order of the
// additions is fixed.  Chunks hold at least 4 blocks (256 rows) each; at most kMaxChunks.
DensePlan dense_plan(int32_t batch, int32_t n_in, int32_t n_out) {
  DensePlan pl;
  pl.tiles = (n_out + kTileCols - 1) / kTileCols;
  pl.groups = (batch + kGroupRows - 1) / kGroupRows;
  const int64_t blocks = ((int64_t)n_in + kBlk - 1) / kBlk;
  const int64_t wgs = (int64_t)pl.tiles * pl.groups;
  int64_t s0 = kTargetGroups / (wgs > 0 ? wgs : 1);
  const int64_t smax = blocks / 4;
  if (s0 > smax) s0 = smax;
  if (s0 > kMaxChunks) s0 = kMaxChunks;
  if (s0 < 1) s0 = 1;
  const int64_t per = blocks > 0 ? (blocks + s0 - 1) / s0 : 1;  // blocks per chunk
  pl.chunks = blocks > 0 ? (int32_t)((blocks + per - 1) / per) : 1;
  pl.chunk_rows = (int32_t)(per * kBlk);
  return pl;
}

// Workspace: [0, ticket bytes) one counter per (batch group, column tile), zero on entry and
// on return; then the partial sums [S][batch][n_out].
size_t dense_ticket_bytes(const DensePlan& pl) {
  if (pl.chunks <= 1) return 0;
  return ((size_t)pl.tiles * pl.groups * sizeof(uint32_t) + 255) & ~(size_t)255;
}
size_t dense_ws_bytes(const DensePlan& pl, int32_t batch, int32_t n_out) {
  if (pl.chunks <= 1) return 0;
  return dense_ticket_bytes(pl) + (size_t)pl.chunks * batch * n_out * sizeof(float);
}

template <int V>
struct VecF;
template <>
struct VecF<1> { using T = float; };
template <>
struct VecF<2> { using T = float2; };
template <>
struct VecF<4> { using T = float4; };

template <int V>
__device__ __forceinline__ void add_vec(float* acc, const typename VecF<V>::T& x) {
  const float* e = (const float*)&x;
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] += e[v];
}
template <int V>
__device__ __forceinline__ void fma_vec(float* acc, float s, const typename VecF<V>::T& x) {
  const float* e = (const float*)&x;
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] += s * e[v];  // product rounded, then the sum
}

template <typename T, bool kEvent, bool kVec>
__global__ __launch_bounds__(kDB) void k_event_dense(const T* __restrict__ spk, int32_t batch,
                                                     int32_t n_in, const float* __restrict__ W,
                                                     int32_t n_out, float* __restrict__ out,
                                                     DensePlan pl, float* part, uint32_t* tick) {
  using VT = typename VecF<kV>::T;
  constexpr int kRowF4 = kTileCols / 4;             // float4 per block row
  constexpr int kStage = kBlk * kRowF4 / kDB;       // float4 staged per thread per block
  constexpr uint32_t kZeroOff = kBlk * kTileCols * 4;  // byte offset of the zero row
  __shared__ __align__(16) float s_w[2][(kBlk + 1) * kTileCols];  // row kBlk stays zero
  __shared__ __align__(16) uint32_t s_list[kDWaves][kRowsPerWave][kList];
  __shared__ __align__(16) float s_val[kEvent ? 1 : kDWaves][kRowsPerWave][kList];
  __shared__ uint32_t s_last;

  const int32_t per_xcd = gridDim.x / kXcds;  // the grid is a multiple of kXcds
  const int32_t lwg = (int32_t)(blockIdx.x % kXcds) * per_xcd + (int32_t)(blockIdx.x / kXcds);
  if (lwg >= pl.tiles * pl.groups * pl.chunks) return;  // whole workgroup
  const int32_t ct = lwg % pl.tiles;
  const int32_t rest = lwg / pl.tiles;
  const int32_t bg = rest % pl.groups;
  const int32_t kc = rest / pl.groups;
  const int lane = bs_lane();
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / BS_WAVE));
  const int32_t col = ct * kTileCols + lane * kV;
  const int32_t r_lo = kc * pl.chunk_rows;
  const int32_t r_hi = r_lo + pl.chunk_rows < n_in ? r_lo + pl.chunk_rows : n_in;
  const int32_t nblk = (r_hi - r_lo + kBlk - 1) / kBlk;

  for (int x = threadIdx.x; x < kTileCols; x += kDB) {
    s_w[0][kBlk * kTileCols + x] = 0.0f;
    s_w[1][kBlk * kTileCols + x] = 0.0f;
  }

  // staging: float4 q of thread t is element t + q*kDB of the block, row-major
  auto load_block = [&](int32_t k, float4* dst) {
#pragma unroll
    for (int q = 0; q < kStage; ++q) {
      const int e = (int)threadIdx.x + q * kDB;
      const int row = e / kRowF4;
      const int32_t c = ct * kTileCols + (e - row * kRowF4) * 4;
      const int32_t i = r_lo + k * kBlk + row;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (k < nblk && i < r_hi) {
        const float* p = W + (int64_t)i * n_out + c;
        if (kVec) {
          if (c < n_out) v = *(const float4*)p;  // n_out % 4 == 0
        } else {
          if (c < n_out) v.x = p[0];
          if (c + 1 < n_out) v.y = p[1];
          if (c + 2 < n_out) v.z = p[2];
          if (c + 3 < n_out) v.w = p[3];
        }
      }
      dst[q] = v;
    }
  };
  // spikes: lane l of the wave holds input ib + l of each of its batch rows; the load is
  // unconditional (clamped address), the flag says whether the input exists
  auto load_spk = [&](int32_t k, T* dst, bool* ok) {
#pragma unroll
    for (int u = 0; u < kRowsPerWave; ++u) {
      const int32_t b = bg * kGroupRows + wid + kDWaves * u;
      const int32_t i = r_lo + k * kBlk + lane;
      ok[u] = k < nblk && b < batch && i < r_hi;
      dst[u] = spk[ok[u] ? (int64_t)b * n_in + i : 0];
    }
  };

  float acc[kRowsPerWave][kV];
#pragma unroll
  for (int u = 0; u < kRowsPerWave; ++u)
#pragma unroll
    for (int v = 0; v < kV; ++v) acc[u][v] = 0.0f;

  float4 pre[kDepth][kStage];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) load_block(d, pre[d]);
  T sp[kRowsPerWave];
  bool sok[kRowsPerWave];
  load_spk(0, sp, sok);

  for (int32_t k0 = 0; k0 < nblk; k0 += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int32_t k = k0 + d;
      if (k >= nblk) break;  // uniform
      float* sw = s_w[k & 1];
#pragma unroll
      for (int q = 0; q < kStage; ++q) {
        const int e = (int)threadIdx.x + q * kDB;
        const int row = e / kRowF4;
        *(float4*)&sw[row * kTileCols + (e - row * kRowF4) * 4] = pre[d][q];
      }
      // this wave's lists for block k: byte offsets of the active rows, ascending, padded
      // with the zero row to a multiple of 4 (8 entries are always valid).  One LDS write per
      // row for all lanes: an active lane writes its entry at its rank, the first 8 inactive
      // lanes write the padding after the last entry, the others a slot that is never read.
      uint32_t cnt[kRowsPerWave];
#pragma unroll
      for (int u = 0; u < kRowsPerWave; ++u) {
        const bool on = sok[u] && nz(sp[u]);
        const uint64_t m = bs_ballot(on);
        cnt[u] = (uint32_t)__popcll(m);
        const uint32_t below = (uint32_t)bs_rank_below(m);
        const uint32_t idle = (uint32_t)lane - below;  // inactive lanes below this one
        const uint32_t pos = on ? below : (idle < 8 ? cnt[u] + idle : (uint32_t)kDump);
        s_list[wid][u][pos] = on ? (uint32_t)lane * (kTileCols * 4) : kZeroOff;
        if (!kEvent) s_val[kEvent ? 0 : wid][u][pos] = on ? (float)sp[u] : 0.0f;
      }
      // next spikes first, then the next W block: a wait for the spikes never waits for W
      load_spk(k + 1, sp, sok);
      load_block(k + kDepth, pre[d]);
      // read the first 8 entries of each row back now (this wave wrote them), so only the
      // W reads wait behind the barrier
      uint4 e0[kRowsPerWave], e1[kRowsPerWave];
      float4 sv0[kRowsPerWave], sv1[kRowsPerWave];
#pragma unroll
      for (int u = 0; u < kRowsPerWave; ++u) {
        e0[u] = *(const uint4*)&s_list[wid][u][0];
        e1[u] = *(const uint4*)&s_list[wid][u][4];
        if (!kEvent) {
          sv0[u] = *(const float4*)&s_val[kEvent ? 0 : wid][u][0];
          sv1[u] = *(const float4*)&s_val[kEvent ? 0 : wid][u][4];
        }
      }
      __syncthreads();

      const char* wb = (const char*)sw + lane * kV * 4;
      VT x0[kRowsPerWave][4], x1[kRowsPerWave][4];
#pragma unroll
      for (int u = 0; u < kRowsPerWave; ++u) {
        x0[u][0] = *(const VT*)(wb + e0[u].x);
        x0[u][1] = *(const VT*)(wb + e0[u].y);
        x0[u][2] = *(const VT*)(wb + e0[u].z);
        x0[u][3] = *(const VT*)(wb + e0[u].w);
      }
#pragma unroll
      for (int u = 0; u < kRowsPerWave; ++u) {
        if (cnt[u] > 4) {  // uniform
          x1[u][0] = *(const VT*)(wb + e1[u].x);
          x1[u][1] = *(const VT*)(wb + e1[u].y);
          x1[u][2] = *(const VT*)(wb + e1[u].z);
          x1[u][3] = *(const VT*)(wb + e1[u].w);
        }
      }
#pragma unroll
      for (int u = 0; u < kRowsPerWave; ++u) {
        if (kEvent) {
#pragma unroll
          for (int q = 0; q < 4; ++q) add_vec<kV>(acc[u], x0[u][q]);
        } else {
          fma_vec<kV>(acc[u], sv0[u].x, x0[u][0]);
          fma_vec<kV>(acc[u], sv0[u].y, x0[u][1]);
          fma_vec<kV>(acc[u], sv0[u].z, x0[u][2]);
          fma_vec<kV>(acc[u], sv0[u].w, x0[u][3]);
        }
        if (cnt[u] > 4) {
          if (kEvent) {
#pragma unroll
            for (int q = 0; q < 4; ++q) add_vec<kV>(acc[u], x1[u][q]);
          } else {
            fma_vec<kV>(acc[u], sv1[u].x, x1[u][0]);
            fma_vec<kV>(acc[u], sv1[u].y, x1[u][1]);
            fma_vec<kV>(acc[u], sv1[u].z, x1[u][2]);
            fma_vec<kV>(acc[u], sv1[u].w, x1[u][3]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kRowsPerWave; ++u) {
        for (uint32_t j = 8; j < cnt[u]; j += 4) {  // rows with more than 8 events
          const uint4 e = *(const uint4*)&s_list[wid][u][j];
          const VT x1 = *(const VT*)(wb + e.x);
          const VT x2 = *(const VT*)(wb + e.y);
          const VT x3 = *(const VT*)(wb + e.z);
          const VT x4 = *(const VT*)(wb + e.w);
          if (kEvent) {
            add_vec<kV>(acc[u], x1);
            add_vec<kV>(acc[u], x2);
            add_vec<kV>(acc[u], x3);
            add_vec<kV>(acc[u], x4);
          } else {
            const float4 sv = *(const float4*)&s_val[kEvent ? 0 : wid][u][j];
            fma_vec<kV>(acc[u], sv.x, x1);
            fma_vec<kV>(acc[u], sv.y, x2);
            fma_vec<kV>(acc[u], sv.z, x3);
            fma_vec<kV>(acc[u], sv.w, x4);
          }
        }
      }
    }
  }

  auto store_row = [&](float* dst, const float* a) {  // V columns at dst (col < n_out)
#pragma unroll
    for (int v = 0; v < kV; ++v)
      if (col + v < n_out) dst[v] = a[v];
  };
  if (pl.chunks == 1) {
#pragma unroll
    for (int u = 0; u < kRowsPerWave; ++u) {
      const int32_t b = bg * kGroupRows + wid + kDWaves * u;
      if (b < batch) store_row(out + (int64_t)b * n_out + col, acc[u]);
    }
    return;
  }
  // partial sums of this chunk, then a ticket; the last workgroup adds them in chunk order
#pragma unroll
  for (int u = 0; u < kRowsPerWave; ++u) {
    const int32_t b = bg * kGroupRows + wid + kDWaves * u;
    if (b < batch) {
      uint32_t* pp = (uint32_t*)part + ((int64_t)kc * batch + b) * n_out + col;
#pragma unroll
      for (int v = 0; v < kV; ++v)
        if (col + v < n_out)
          __hip_atomic_store(pp + v, __float_as_uint(acc[u][v]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partials are complete at device scope
  __syncthreads();
  uint32_t* tk = tick + (int64_t)bg * pl.tiles + ct;
  if (threadIdx.x == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old + 1 == (uint32_t)pl.chunks ? 1u : 0u;
    if (s_last) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  // every partial of this thread's outputs in flight at once, then the sums in chunk order
  float pv[kMaxChunks][kRowsPerWave][kV];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
#pragma unroll
    for (int u = 0; u < kRowsPerWave; ++u) {
      const int32_t b = bg * kGroupRows + wid + kDWaves * u;
      const uint32_t* pp = (const uint32_t*)part + ((int64_t)c * batch + b) * n_out + col;
#pragma unroll
      for (int v = 0; v < kV; ++v) {
        pv[c][u][v] = acc[u][v];
        if (c < pl.chunks && c != kc && b < batch && col + v < n_out)
          pv[c][u][v] = __uint_as_float(
              __hip_atomic_load(pp + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kRowsPerWave; ++u) {
    const int32_t b = bg * kGroupRows + wid + kDWaves * u;
    float tot[kV];
#pragma unroll
    for (int v = 0; v < kV; ++v) {
      tot[v] = pv[0][u][v];
#pragma unroll
      for (int c = 1; c < kMaxChunks; ++c)
        if (c < pl.chunks) tot[v] = tot[v] + pv[c][u][v];
    }
    if (b < batch) store_row(out + (int64_t)b * n_out + col, tot);
  }
}

template <typename T>
int launch(const T* spk, int32_t batch, int32_t n_in, const float* W, int32_t n_out, bool ev,
           float* out, void* ws, size_t ws_bytes, hipStream_t s) {
  const DensePlan pl = dense_plan(batch, n_in, n_out);
  float* part = nullptr;
  uint32_t* tick = nullptr;
  if (pl.chunks > 1) {
    const size_t need = dense_ws_bytes(pl, batch, n_out);
    if (ws == nullptr || ws_bytes < need) {
      bs_set_error("bs_event_dense_f32: workspace of %zu bytes needed (got %zu)", need,
                   ws == nullptr ? (size_t)0 : ws_bytes);
      return BS_ERR_INVALID;
    }
    tick = (uint32_t*)ws;
    part = (float*)((char*)ws + dense_ticket_bytes(pl));
  }
  int64_t g = (int64_t)pl.tiles * pl.groups * pl.chunks;
  if (g > INT32_MAX - kXcds) {
    bs_set_error("bs_event_dense_f32: %lld workgroups exceed the grid limit", (long long)g);
    return BS_ERR_INVALID;
  }
  g = (g + kXcds - 1) / kXcds * kXcds;
  const bool vec = n_out % 4 == 0 && ((uintptr_t)W & 15) == 0;
#define BS_DENSE(E, VV)                                                                 \
  k_event_dense<T, E, VV><<<(int)g, kDB, 0, s>>>(spk, batch, n_in, W, n_out, out, pl, part, \
                                                 tick)
  if (ev) { if (vec) BS_DENSE(true, true); else BS_DENSE(true, false); }
  else { if (vec) BS_DENSE(false, true); else BS_DENSE(false, false); }
#undef BS_DENSE
  BS_CHECK_LAUNCH();
  return BS_OK;
}

// ---- reverse mode: y[b] = sum_i x[b,i] * W[i] (x = spike value, 1 for byte spikes) ----

// grad_x[b,i] = sum_j g[b,j] * W[i,j]: one wave per (input row i, kGb batch rows); lanes
// stride the columns (16-byte loads of W and g), then each of the kGb sums is reduced across
// the wave.
constexpr int kGb = 8;
template <int V>
__global__ __launch_bounds__(kBlock) void k_dense_gx(int32_t batch, int32_t n_in,
                                                     const float* __restrict__ W, int32_t n_out,
                                                     const float* __restrict__ g,
                                                     float* __restrict__ gx) {
  const int lane = bs_lane();
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE;
  const int32_t bgroups = (batch + kGb - 1) / kGb;
  if (wave >= (int64_t)n_in * bgroups) return;
  const int32_t i = (int32_t)(wave / bgroups);
  const int32_t b0 = (int32_t)(wave - (int64_t)i * bgroups) * kGb;
  float acc[kGb];
#pragma unroll
  for (int u = 0; u < kGb; ++u) acc[u] = 0.0f;
  const float* wr = W + (int64_t)i * n_out;
  for (int32_t j = lane * V; j < n_out; j += BS_WAVE * V) {
    float wv[V];
    if (V == 4) {
      const float4 q = *(const float4*)(wr + j);
      wv[0] = q.x;
      wv[V > 1 ? 1 : 0] = q.y;
      wv[V > 2 ? 2 : 0] = q.z;
      wv[V > 3 ? 3 : 0] = q.w;
    } else {
      wv[0] = wr[j];
    }
#pragma unroll
    for (int u = 0; u < kGb; ++u) {
      if (b0 + u < batch) {
        const float* gr = g + (int64_t)(b0 + u) * n_out + j;
        if (V == 4) {
          const float4 q = *(const float4*)gr;
          acc[u] = bs_fma(q.x, wv[0], acc[u]);
          acc[u] = bs_fma(q.y, wv[V > 1 ? 1 : 0], acc[u]);
          acc[u] = bs_fma(q.z, wv[V > 2 ? 2 : 0], acc[u]);
          acc[u] = bs_fma(q.w, wv[V > 3 ? 3 : 0], acc[u]);
        } else {
          acc[u] = bs_fma(gr[0], wv[0], acc[u]);
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kGb; ++u) {
#pragma unroll
    for (int o = BS_WAVE / 2; o > 0; o >>= 1) acc[u] += __shfl_xor(acc[u], o);
  }
  if (lane < kGb && b0 + lane < batch) {
    float v = acc[0];
#pragma unroll
    for (int u = 1; u < kGb; ++u) v = lane == u ? acc[u] : v;
    gx[(int64_t)(b0 + lane) * n_in + i] = v;
  }
}

// grad_x = g W^T on the matrix cores (fp32 v_mfma_f32_16x16x4f32) when n_out is a multiple
// of 16 and W and g are 16-byte aligned: a workgroup owns 16 input rows x 64 batch rows; its 4
// waves split the n_out sum into 4 ranges of 16-wide blocks, and each wave accumulates the
// four 16-row batch tiles over its range.  Per block, lane l loads 4 consecutive k of W row
// i0 + l % 16 and of the g rows, so instruction t of the block takes k = k0 + 4 (l / 16) + t
// for both operands (the instruction sums over l / 16; the four instructions cover the 16 k).
// Rows past n_in or batch load a clamped in-bounds row and are never stored.  The waves'
// partial tiles meet in LDS and are added in wave order: fp32 sums in a fixed order, not the
// row-sequential order of k_dense_gx (the same results within fp32 rounding of the sum).
// At 64 x 4096 x 4096: 172 us for k_dense_gx, 42.5 us here.  What bounds it (timing copies
// with loads left out): the products alone take 18.5 us, with W's loads 25.5, with g's 34.9:
// every 16-row tile reads all of g from L2 (256 MB per call), which only wider tiles with a
// split-K reduction across workgroups would cut.
constexpr int kMxW = 4;          // waves per workgroup (n_out ranges)
constexpr int kMxG = 2;          // 16-wide k blocks per pipeline stage
typedef float v4f __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kMxW * BS_WAVE) void k_dense_gx_mfma(int32_t batch, int32_t n_in,
                                                                  const float* __restrict__ W,
                                                                  int32_t n_out,
                                                                  const float* __restrict__ g,
                                                                  float* __restrict__ gx) {
  __shared__ v4f s_part[kMxW][4][BS_WAVE];  // 16 KiB
  const int lane = bs_lane();
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / BS_WAVE));
  const int64_t i0 = (int64_t)blockIdx.x * 16;
  const int32_t b0 = (int32_t)blockIdx.y * 64;
  const int32_t KB = n_out / 16;
  const int32_t k_lo = (int32_t)((int64_t)KB * wid / kMxW);
  const int32_t k_hi = (int32_t)((int64_t)KB * (wid + 1) / kMxW);
  const int64_t wi = i0 + (lane & 15) < n_in ? i0 + (lane & 15) : (int64_t)n_in - 1;
  const int kq = 4 * (lane >> 4);
  const float* wp = W + wi * n_out + kq;
  const float* gp[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int32_t b = b0 + 16 * mt + (lane & 15);
    gp[mt] = g + (int64_t)(b < batch ? b : batch - 1) * n_out + kq;
  }
  v4f acc[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) acc[mt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // one stage: kMxG blocks (blocks at or past k_hi load zeros and add nothing)
  auto load = [&](int32_t kb, v4f (&wv)[kMxG], v4f (&gv)[kMxG][4]) {
#pragma unroll
    for (int u = 0; u < kMxG; ++u) {
      const bool ok = kb + u < k_hi;
      const int64_t o = (int64_t)(kb + u) * 16;
      wv[u] = ok ? *(const v4f*)(wp + o) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        gv[u][mt] = ok ? *(const v4f*)(gp[mt] + o) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  auto mult = [&](const v4f (&wv)[kMxG], const v4f (&gv)[kMxG][4]) {
#pragma unroll
    for (int u = 0; u < kMxG; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)   // consecutive products update different tiles
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(gv[u][mt][t], wv[u][t], acc[mt], 0, 0, 0);
  };
  if (k_lo < k_hi) {
    // two register stages: the next stage's loads are issued (kept together, ahead of the
    // products, by the scheduling barriers) before the current stage is multiplied
    auto sched = [] { __builtin_amdgcn_sched_barrier(0); };
    v4f wa[kMxG], ga[kMxG][4], wb[kMxG], gb[kMxG][4];
    load(k_lo, wa, ga);
    for (int32_t kb = k_lo; kb < k_hi; kb += 2 * kMxG) {
      sched(); load(kb + kMxG, wb, gb); sched();
      mult(wa, ga);
      sched(); load(kb + 2 * kMxG, wa, ga); sched();
      mult(wb, gb);
    }
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) s_part[wid][mt][lane] = acc[mt];
  __syncthreads();
  // wave w adds the 4 waves' partials of batch tile w in wave order; lane l holds rows
  // 4 (l / 16) + r of the tile, column l % 16
  const int mt = wid;
  v4f v = s_part[0][mt][lane];
#pragma unroll
  for (int w = 1; w < kMxW; ++w) v += s_part[w][mt][lane];
  const int64_t i = i0 + (lane & 15);
  if (i < n_in) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t b = b0 + 16 * mt + 4 * (lane >> 4) + r;
      if (b < batch) gx[(int64_t)b * n_in + i] = v[r];
    }
  }
}

// grad_W[i,j] = sum_b x[b,i] * g[b,j]: one wave per (input row i, kGwTiles tiles of 64*V
// columns); the wave ballots the batch rows whose spike i is nonzero (64 at a time; the first
// 64 once for all its tiles) and adds their g rows in ascending b.  Every element of grad_W is
// written (rows no spike selects get 0).  64 x 4096 x 4096: 24.5 us with one tile per wave,
// 21.9 with 4 (16: 37 us, too few waves; loading up to 4 selected g rows together: 22.7).
constexpr int kGwTiles = 4;
template <typename T, int V>
__global__ __launch_bounds__(kBlock) void k_dense_gw(const T* __restrict__ spk, int32_t batch,
                                                     int32_t n_in, int32_t n_out,
                                                     const float* __restrict__ g,
                                                     float* __restrict__ gw) {
  const int lane = bs_lane();
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE;
  const int32_t tiles = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
  constexpr int kTpw = kGwTiles;
  const int32_t tgroups = (tiles + kTpw - 1) / kTpw;
  if (wave >= (int64_t)n_in * tgroups) return;
  const int32_t i = (int32_t)(wave / tgroups);
  const int32_t tg = (int32_t)(wave - (int64_t)i * tgroups);
  // batch <= 64: the row's spike column and its ballot once for all the wave's tiles
  const float xv0 = lane < batch ? (float)spk[(int64_t)lane * n_in + i] : 0.0f;
  const uint64_t m0 = bs_ballot(xv0 != 0.0f);
  for (int32_t tt = 0; tt < kTpw; ++tt) {
    const int32_t t = tg * kTpw + tt;
    if (t >= tiles) break;
    const int32_t j0 = t * BS_WAVE * V + lane * V;
    const bool live = j0 < n_out;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0f;
    for (int32_t bb = 0; bb < batch; bb += BS_WAVE) {
      const float xv = bb == 0 ? xv0 : (bb + lane < batch ? (float)spk[(int64_t)(bb + lane) * n_in + i] : 0.0f);
      uint64_t m = bb == 0 ? m0 : bs_ballot(xv != 0.0f);
      while (m) {
        const int bit = __builtin_ctzll(m);
        m &= m - 1;
        const float xb = __shfl(xv, bit);
        if (live) {
          const float* gr = g + (int64_t)(bb + bit) * n_out + j0;
          if (V == 4) {
            const float4 q = *(const float4*)gr;
            acc[0] = bs_fma(xb, q.x, acc[0]);
            acc[V > 1 ? 1 : 0] = bs_fma(xb, q.y, acc[V > 1 ? 1 : 0]);
            acc[V > 2 ? 2 : 0] = bs_fma(xb, q.z, acc[V > 2 ? 2 : 0]);
            acc[V > 3 ? 3 : 0] = bs_fma(xb, q.w, acc[V > 3 ? 3 : 0]);
          } else {
            acc[0] = bs_fma(xb, gr[0], acc[0]);
          }
        }
      }
    }
    if (live) {
      float* o = gw + (int64_t)i * n_out + j0;
      if (V == 4) *(float4*)o = make_float4(acc[0], acc[V > 1 ? 1 : 0], acc[V > 2 ? 2 : 0], acc[V > 3 ? 3 : 0]);
      else o[0] = acc[0];
    }
  }
}

}  // namespace

int bs_fill_f32(float* p, int64_t n, float v, hipStream_t s);

extern "C" int bs_event_dense_chunks(int32_t batch, int32_t n_in, int32_t n_out,
                                     int32_t* chunk_rows) {
  bs_clear_error();
  BS_CHECK_ARG(batch >= 0 && n_in >= 0 && n_out >= 0, "bs_event_dense_chunks: negative size");
  const DensePlan pl = dense_plan(batch, n_in, n_out);
  if (chunk_rows) *chunk_rows = pl.chunk_rows;
  return pl.chunks;
}

extern "C" size_t bs_event_dense_workspace_size(int32_t batch, int32_t n_in, int32_t n_out) {
  bs_clear_error();
  if (batch <= 0 || n_in <= 0 || n_out <= 0) return 0;
  return dense_ws_bytes(dense_plan(batch, n_in, n_out), batch, n_out);
}

extern "C" size_t bs_event_dense_ticket_bytes(int32_t batch, int32_t n_in, int32_t n_out) {
  bs_clear_error();
  if (batch <= 0 || n_in <= 0 || n_out <= 0) return 0;
  return dense_ticket_bytes(dense_plan(batch, n_in, n_out));
}

extern "C" int bs_event_dense_f32(const void* spk, int32_t spk_dtype, int32_t batch, int32_t n_in,
                                  const float* W, int32_t n_out, int32_t float_as_event,
                                  float* out, void* workspace, size_t workspace_bytes,
                                  bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(batch >= 0 && n_in >= 0 && n_out >= 0, "bs_event_dense_f32: negative size");
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_event_dense_f32: unknown spike dtype %d", spk_dtype);
  if (batch == 0 || n_out == 0) return BS_OK;
  BS_CHECK_ARG(out != nullptr, "bs_event_dense_f32: out is NULL");
  hipStream_t s = bs_stream(stream);
  if (n_in == 0) return bs_fill_f32(out, (int64_t)batch * n_out, 0.0f, s);
  BS_CHECK_ARG(spk && W, "bs_event_dense_f32: NULL pointer");
  const bool ev = float_as_event != 0;
  if (spk_dtype == BS_SPK_U8)
    return launch((const uint8_t*)spk, batch, n_in, W, n_out, ev, out, workspace,
                  workspace_bytes, s);
  return launch((const float*)spk, batch, n_in, W, n_out, ev, out, workspace, workspace_bytes,
                s);
}

extern "C" int bs_event_dense_vjp_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                      int32_t n_in, const float* W, int32_t n_out,
                                      const float* grad_out, float* grad_spk, float* grad_W,
                                      bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(batch >= 0 && n_in >= 0 && n_out >= 0, "bs_event_dense_vjp_f32: negative size");
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_event_dense_vjp_f32: unknown spike dtype %d", spk_dtype);
  hipStream_t s = bs_stream(stream);
  if (n_in == 0) return BS_OK;
  if (n_out == 0 || batch == 0) {  // empty sums
    if (grad_spk) {
      int rc = bs_fill_f32(grad_spk, (int64_t)batch * n_in, 0.0f, s);
      if (rc) return rc;
    }
    if (grad_W) return bs_fill_f32(grad_W, (int64_t)n_in * n_out, 0.0f, s);
    return BS_OK;
  }
  BS_CHECK_ARG(grad_out != nullptr, "bs_event_dense_vjp_f32: grad_out is NULL");
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = n_out % 4 == 0 && al(grad_out);
  if (grad_spk) {
    BS_CHECK_ARG(W != nullptr, "bs_event_dense_vjp_f32: W is NULL");
    const int64_t waves = (int64_t)n_in * ((batch + kGb - 1) / kGb);
    const int g = (int)((waves + (kBlock / BS_WAVE) - 1) / (kBlock / BS_WAVE));
    if (n_out % 16 == 0 && al(W) && al(grad_out) && (batch + 63) / 64 <= 65535) {
      const dim3 gg((unsigned)((n_in + 15) / 16), (unsigned)((batch + 63) / 64));
      k_dense_gx_mfma<<<gg, kMxW * BS_WAVE, 0, s>>>(batch, n_in, W, n_out, grad_out, grad_spk);
    } else if (vec && al(W)) {
      k_dense_gx<4><<<g, kBlock, 0, s>>>(batch, n_in, W, n_out, grad_out, grad_spk);
    } else {
      k_dense_gx<1><<<g, kBlock, 0, s>>>(batch, n_in, W, n_out, grad_out, grad_spk);
    }
    BS_CHECK_LAUNCH();
  }
  if (grad_W) {
    BS_CHECK_ARG(spk != nullptr, "bs_event_dense_vjp_f32: spk is NULL");
    const bool v4 = vec && al(grad_W);
    const int V = v4 ? 4 : 1;
    const int64_t tiles_ = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
    const int64_t waves = (int64_t)n_in * ((tiles_ + kGwTiles - 1) / kGwTiles);
    const int g = (int)((waves + (kBlock / BS_WAVE) - 1) / (kBlock / BS_WAVE));
#define BS_GW(T, VV) \
  k_dense_gw<T, VV><<<g, kBlock, 0, s>>>((const T*)spk, batch, n_in, n_out, grad_out, grad_W)
    if (spk_dtype == BS_SPK_U8) { if (v4) BS_GW(uint8_t, 4); else BS_GW(uint8_t, 1); }
    else { if (v4) BS_GW(float, 4); else BS_GW(float, 1); }
#undef BS_GW
    BS_CHECK_LAUNCH();
  }
  return BS_OK;
}

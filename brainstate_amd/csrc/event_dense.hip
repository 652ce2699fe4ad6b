// N2c: batched event x dense weight (EventLinear).
//
// One wave per (batch row b, tile of 64*V output columns).  Each lane turns 64 consecutive
// spikes of row b into a 64-bit mask (coalesced 16-byte loads); the wave walks the masks in
// order and streams the active inputs kBatch at a time across mask boundaries: kBatch
// coalesced row segments of W (128-bit loads when V = 4) are in flight before the first add,
// so a 5 %-dense row costs about (active inputs / kBatch) memory round trips, not one per 64
// inputs.  Each lane adds its V columns in
// ascending input order, the order of a sequential reference loop, so results are
// bit-reproducible.
//
// XCD-aware placement: a row segment of W is needed by every batch row whose spike selects
// it, and those waves all read the tile's segments in ascending input order.  Waves are
// therefore numbered tile-major (all batch rows of a tile consecutive) and consecutive
// logical workgroups are placed on the same XCD (workgroups are dispatched to the 8 XCDs
// round-robin), so the batch rows of a tile share that XCD's L2 and each segment is fetched
// from memory about once per step instead of once per batch row that uses it.
#include "bs_math.h"
#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kBatch = 16;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2


// Spike byte/float -> event flag (any nonzero value is an event).
__device__ __forceinline__ bool nz(uint8_t x) { return x != 0; }
__device__ __forceinline__ bool nz(float x) { return x != 0.0f; }

// Mask of the 64 inputs [i0, i0 + 64) of one spike row, built by one lane from coalesced
// 16-byte loads (bit k = input i0 + k; inputs at or past n_in are 0).
template <typename T>
__device__ __forceinline__ uint64_t lane_mask(const T* row, int32_t i0, int32_t n_in) {
  uint64_t m = 0;
  if (i0 + 64 <= n_in && (((uintptr_t)(row + i0)) & 15) == 0) {
    constexpr int kPer = 16 / sizeof(T);  // inputs per 16-byte load
#pragma unroll
    for (int c = 0; c < 64; c += kPer) {
      const uint4 q = *(const uint4*)(row + i0 + c);
      const T* e = (const T*)&q;
#pragma unroll
      for (int k = 0; k < kPer; ++k) m |= (uint64_t)nz(e[k]) << (c + k);
    }
  } else {
    for (int k = 0; k < 64 && i0 + k < n_in; ++k) m |= (uint64_t)nz(row[i0 + k]) << k;
  }
  return m;
}

// 64-bit value of lane l (l wave-uniform).
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

template <typename T, int V, bool kEvent>
__global__ __launch_bounds__(kBlock) void k_event_dense(const T* __restrict__ spk, int32_t batch,
                                                        int32_t n_in, const float* __restrict__ W,
                                                        int32_t n_out, float* __restrict__ out) {
  const int lane = bs_lane();
  const int32_t per_xcd = gridDim.x / kXcds;  // the grid is a multiple of kXcds
  const int64_t lwg = (int64_t)(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  const int64_t wave = (lwg * kBlock + threadIdx.x) / BS_WAVE;  // tile-major wave number
  const int32_t tiles = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
  if (wave >= (int64_t)batch * tiles) return;
  const int32_t t = (int32_t)(wave / batch);
  const int32_t b = (int32_t)(wave - (int64_t)t * batch);
  const int32_t j0 = t * BS_WAVE * V + lane * V;
  const bool live = j0 < n_out;
  const T* srow = spk + (int64_t)b * n_in;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  // Inputs in spans of 64 groups of 64: lane l holds the mask of group l of the span; the
  // wave walks the groups in order (readlane, no memory access) and fills kBatch row slots
  // across group boundaries before issuing their loads.
  for (int32_t s0 = 0; s0 < n_in; s0 += BS_WAVE * BS_WAVE) {
    const uint64_t mine = lane_mask(srow, s0 + lane * BS_WAVE, n_in);
    const int ng = (n_in - s0 + BS_WAVE - 1) / BS_WAVE < BS_WAVE
                       ? (n_in - s0 + BS_WAVE - 1) / BS_WAVE : BS_WAVE;
    int g = 0;
    uint64_t m = readlane64(mine, 0);
    for (;;) {
      int32_t r[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        while (m == 0 && g + 1 < ng) m = readlane64(mine, ++g);
        r[u] = -1;
        if (m) {
          r[u] = s0 + g * BS_WAVE + (int32_t)__builtin_ctzll(m);
          m &= m - 1;
        }
      }
      if (r[0] < 0) break;
      float x[kBatch][V];
      float sc[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        sc[u] = 1.0f;
        if (r[u] >= 0) {
          if (!kEvent) sc[u] = (float)srow[r[u]];
          if (live) {
            const float* wr = W + (int64_t)r[u] * n_out + j0;
            if (V == 4) {
              const float4 q = *(const float4*)wr;
              x[u][0] = q.x;
              x[u][V > 1 ? 1 : 0] = q.y;
              x[u][V > 2 ? 2 : 0] = q.z;
              x[u][V > 3 ? 3 : 0] = q.w;
            } else if (V == 2) {
              const float2 q = *(const float2*)wr;
              x[u][0] = q.x;
              x[u][V > 1 ? 1 : 0] = q.y;
            } else {
              x[u][0] = *wr;
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (r[u] >= 0 && live) {
#pragma unroll
          for (int v = 0; v < V; ++v) acc[v] += kEvent ? x[u][v] : sc[u] * x[u][v];
        }
      }
    }
  }
  if (live) {
    float* o = out + (int64_t)b * n_out + j0;
    if (V == 4) {
      *(float4*)o = make_float4(acc[0], acc[V > 1 ? 1 : 0], acc[V > 2 ? 2 : 0], acc[V > 3 ? 3 : 0]);
    } else if (V == 2) {
      *(float2*)o = make_float2(acc[0], acc[V > 1 ? 1 : 0]);
    } else {
      o[0] = acc[0];
    }
  }
}

template <typename T, int V>
int launch_v(const T* spk, int32_t batch, int32_t n_in, const float* W, int32_t n_out, bool ev,
             float* out, hipStream_t s) {
  const int64_t tiles = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
  const int64_t waves = (int64_t)batch * tiles;
  int64_t g = (waves + (kBlock / BS_WAVE) - 1) / (kBlock / BS_WAVE);
  g = (g + kXcds - 1) / kXcds * kXcds;
  if (ev) k_event_dense<T, V, true><<<(int)g, kBlock, 0, s>>>(spk, batch, n_in, W, n_out, out);
  else k_event_dense<T, V, false><<<(int)g, kBlock, 0, s>>>(spk, batch, n_in, W, n_out, out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

// Columns per lane: as many as alignment allows while the launch still has about 16 waves per
// CU (4 per SIMD) to overlap the latency of the row loads.
template <typename T>
int launch(const T* spk, int32_t batch, int32_t n_in, const float* W, int32_t n_out, bool ev,
           float* out, hipStream_t s) {
  const auto al = [&](int v) {
    return n_out % v == 0 && ((uintptr_t)W & (4 * v - 1)) == 0 &&
           ((uintptr_t)out & (4 * v - 1)) == 0;
  };
  const int64_t want = (int64_t)4 * bs_num_cus();
  const auto waves = [&](int v) { return (int64_t)batch * ((n_out + BS_WAVE * v - 1) / (BS_WAVE * v)); };
  if (al(4) && waves(4) >= want) return launch_v<T, 4>(spk, batch, n_in, W, n_out, ev, out, s);
  if (al(2) && waves(2) >= want) return launch_v<T, 2>(spk, batch, n_in, W, n_out, ev, out, s);
  return launch_v<T, 1>(spk, batch, n_in, W, n_out, ev, out, s);
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

// grad_W[i,j] = sum_b x[b,i] * g[b,j]: one wave per (input row i, 64*V columns); the wave
// ballots the batch rows whose spike i is nonzero (64 at a time) and adds their g rows in
// ascending b.  Every element of grad_W is written (rows no spike selects get 0).
template <typename T, int V>
__global__ __launch_bounds__(kBlock) void k_dense_gw(const T* __restrict__ spk, int32_t batch,
                                                     int32_t n_in, int32_t n_out,
                                                     const float* __restrict__ g,
                                                     float* __restrict__ gw) {
  const int lane = bs_lane();
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE;
  const int32_t tiles = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
  if (wave >= (int64_t)n_in * tiles) return;
  const int32_t i = (int32_t)(wave / tiles);
  const int32_t j0 = (int32_t)(wave - (int64_t)i * tiles) * BS_WAVE * V + lane * V;
  const bool live = j0 < n_out;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  for (int32_t bb = 0; bb < batch; bb += BS_WAVE) {
    const float xv = bb + lane < batch ? (float)spk[(int64_t)(bb + lane) * n_in + i] : 0.0f;
    uint64_t m = bs_ballot(xv != 0.0f);
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

}  // namespace

int bs_fill_f32(float* p, int64_t n, float v, hipStream_t s);

extern "C" int bs_event_dense_f32(const void* spk, int32_t spk_dtype, int32_t batch, int32_t n_in,
                                  const float* W, int32_t n_out, int32_t float_as_event,
                                  float* out, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(batch >= 0 && n_in >= 0 && n_out >= 0, "bs_event_dense_f32: negative size");
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_event_dense_f32: unknown spike dtype %d", spk_dtype);
  if (batch == 0 || n_out == 0) return BS_OK;
  BS_CHECK_ARG(out != nullptr, "bs_event_dense_f32: out is NULL");
  hipStream_t s = bs_stream(stream);
  if (n_in == 0) return bs_fill_f32(out, (int64_t)batch * n_out, 0.0f, s);
  BS_CHECK_ARG(spk && W, "bs_event_dense_f32: NULL pointer");
  if (spk_dtype == BS_SPK_U8)
    return launch((const uint8_t*)spk, batch, n_in, W, n_out, float_as_event != 0, out, s);
  return launch((const float*)spk, batch, n_in, W, n_out, float_as_event != 0, out, s);
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
    if (vec && al(W)) k_dense_gx<4><<<g, kBlock, 0, s>>>(batch, n_in, W, n_out, grad_out, grad_spk);
    else k_dense_gx<1><<<g, kBlock, 0, s>>>(batch, n_in, W, n_out, grad_out, grad_spk);
    BS_CHECK_LAUNCH();
  }
  if (grad_W) {
    BS_CHECK_ARG(spk != nullptr, "bs_event_dense_vjp_f32: spk is NULL");
    const bool v4 = vec && al(grad_W);
    const int V = v4 ? 4 : 1;
    const int64_t waves = (int64_t)n_in * ((n_out + BS_WAVE * V - 1) / (BS_WAVE * V));
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

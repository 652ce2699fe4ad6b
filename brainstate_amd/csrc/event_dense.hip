// N2c: batched event x dense weight (EventLinear).
//
// One wave per (batch row b, tile of 64*V output columns).  The wave reads 64 spikes of row b
// per step (one byte or float per lane) and ballots them into a mask; the active inputs of
// the mask are then streamed kBatch at a time: kBatch coalesced row segments of W (128-bit
// loads when V = 4) are in flight before the first add.  Each lane adds its V columns in
// ascending input order, the order of a sequential reference loop, so results are
// bit-reproducible.
#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kBatch = 8;

__device__ __forceinline__ float spk_val(const uint8_t* p, int64_t i) { return (float)p[i]; }
__device__ __forceinline__ float spk_val(const float* p, int64_t i) { return p[i]; }

template <typename T, int V, bool kEvent>
__global__ __launch_bounds__(kBlock) void k_event_dense(const T* __restrict__ spk, int32_t batch,
                                                        int32_t n_in, const float* __restrict__ W,
                                                        int32_t n_out, float* __restrict__ out) {
  const int lane = bs_lane();
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE;
  const int32_t tiles = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
  if (wave >= (int64_t)batch * tiles) return;
  const int32_t b = (int32_t)(wave / tiles);
  const int32_t t = (int32_t)(wave - (int64_t)b * tiles);
  const int32_t j0 = t * BS_WAVE * V + lane * V;
  const bool live = j0 < n_out;
  const T* srow = spk + (int64_t)b * n_in;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  for (int32_t i0 = 0; i0 < n_in; i0 += BS_WAVE) {
    const int32_t i = i0 + lane;
    const float sv = i < n_in ? spk_val(srow, i) : 0.0f;
    uint64_t m = bs_ballot(sv != 0.0f);
    while (m) {
      int32_t r[kBatch];
      float sc[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        r[u] = -1;
        sc[u] = 1.0f;
        if (m) {
          const int bit = __builtin_ctzll(m);
          m &= m - 1;
          r[u] = i0 + bit;
          if (!kEvent) sc[u] = __shfl(sv, bit);
        }
      }
      float x[kBatch][V];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (r[u] >= 0 && live) {
          const float* wr = W + (int64_t)r[u] * n_out + j0;
          if (V == 4) {
            const float4 q = *(const float4*)wr;
            x[u][0] = q.x;
            x[u][V > 1 ? 1 : 0] = q.y;
            x[u][V > 2 ? 2 : 0] = q.z;
            x[u][V > 3 ? 3 : 0] = q.w;
          } else {
            x[u][0] = *wr;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (r[u] >= 0) {
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
    } else {
      o[0] = acc[0];
    }
  }
}

template <typename T>
int launch(const T* spk, int32_t batch, int32_t n_in, const float* W, int32_t n_out, bool ev,
           float* out, hipStream_t s) {
  const bool vec = (n_out % 4 == 0) && (((uintptr_t)W & 15) == 0) && (((uintptr_t)out & 15) == 0);
  const int V = vec ? 4 : 1;
  const int64_t tiles = (n_out + BS_WAVE * V - 1) / (BS_WAVE * V);
  const int64_t waves = (int64_t)batch * tiles;
  const int g = (int)((waves + (kBlock / BS_WAVE) - 1) / (kBlock / BS_WAVE));
  if (vec) {
    if (ev) k_event_dense<T, 4, true><<<g, kBlock, 0, s>>>(spk, batch, n_in, W, n_out, out);
    else k_event_dense<T, 4, false><<<g, kBlock, 0, s>>>(spk, batch, n_in, W, n_out, out);
  } else {
    if (ev) k_event_dense<T, 1, true><<<g, kBlock, 0, s>>>(spk, batch, n_in, W, n_out, out);
    else k_event_dense<T, 1, false><<<g, kBlock, 0, s>>>(spk, batch, n_in, W, n_out, out);
  }
  BS_CHECK_LAUNCH();
  return BS_OK;
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

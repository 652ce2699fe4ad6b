// Ring-buffer delay: the device side of brainstate's Delay (brainstate/nn/_delay.py:399-957).
//
// The history is [length][slot_elems] elements laid out slot-major, so a write is one
// contiguous copy of the current value into its slot and a scalar-delay read is one contiguous
// copy out of a slot.  Reads with per-element delays (vector delays registered with index
// arrays, :762-790 with fancy indexing) gather element j from slot (cur - steps[j]) mod length
// at column cols[j].  Continuous-time reads blend up to four slots with host-computed weights
// (linear, Catmull-Rom, Hermite and Lagrange taps, :163-338), summed left to right in fp32.
#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kMaxTaps = 4;

__global__ __launch_bounds__(kBlock) void k_copy16(const uint4* __restrict__ src,
                                                   uint4* __restrict__ dst, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * kBlock)
    dst[i] = src[i];
}

__global__ __launch_bounds__(kBlock) void k_copy1(const uint8_t* __restrict__ src,
                                                  uint8_t* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock)
    dst[i] = src[i];
}

__device__ __forceinline__ int64_t ring_slot(int64_t cur, int64_t step, int64_t length) {
  const int64_t r = (cur - step) % length;
  return r < 0 ? r + length : r;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_gather(const T* __restrict__ hist, int32_t length,
                                                   int64_t slot_elems, int32_t cur, int32_t step,
                                                   const int32_t* __restrict__ steps,
                                                   const int64_t* __restrict__ cols, int64_t n_out,
                                                   T* __restrict__ out) {
  for (int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x; j < n_out;
       j += (int64_t)gridDim.x * kBlock) {
    const int64_t slot = ring_slot(cur, steps ? steps[j] : step, length);
    const int64_t col = cols ? cols[j] : j;
    out[j] = hist[slot * slot_elems + col];
  }
}

struct Taps {
  int32_t n;
  int32_t slot[kMaxTaps];
  float w[kMaxTaps];
};

__global__ __launch_bounds__(kBlock) void k_taps(const float* __restrict__ hist,
                                                 int64_t slot_elems, Taps tp,
                                                 const int64_t* __restrict__ cols, int64_t n_out,
                                                 float* __restrict__ out) {
  for (int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x; j < n_out;
       j += (int64_t)gridDim.x * kBlock) {
    const int64_t col = cols ? cols[j] : j;
    float acc = tp.w[0] * hist[(int64_t)tp.slot[0] * slot_elems + col];
    for (int q = 1; q < tp.n; ++q) acc = acc + tp.w[q] * hist[(int64_t)tp.slot[q] * slot_elems + col];
    out[j] = acc;
  }
}

int grid_for(int64_t n) {
  int64_t g = (n + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)bs_num_cus() * 16;
  if (g > cap) g = cap;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace

extern "C" int bs_delay_write(void* hist, int32_t length, int64_t slot_bytes, int32_t slot,
                              const void* src, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(hist && src, "bs_delay_write: NULL pointer");
  BS_CHECK_ARG(length > 0 && slot_bytes >= 0, "bs_delay_write: bad sizes length=%d bytes=%lld",
               length, (long long)slot_bytes);
  BS_CHECK_ARG(slot >= 0 && slot < length, "bs_delay_write: slot %d outside [0, %d)", slot,
               length);
  if (slot_bytes == 0) return BS_OK;
  hipStream_t s = bs_stream(stream);
  uint8_t* dst = (uint8_t*)hist + (int64_t)slot * slot_bytes;
  const uint8_t* sp = (const uint8_t*)src;
  if ((((uintptr_t)dst | (uintptr_t)sp | (uintptr_t)slot_bytes) & 15) == 0) {
    const int64_t n16 = slot_bytes / 16;
    k_copy16<<<grid_for(n16), kBlock, 0, s>>>((const uint4*)sp, (uint4*)dst, n16);
  } else {
    k_copy1<<<grid_for(slot_bytes), kBlock, 0, s>>>(sp, dst, slot_bytes);
  }
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_delay_gather(const void* hist, int32_t length, int64_t slot_elems,
                               int32_t elem_bytes, int32_t cur, int32_t step,
                               const int32_t* steps, const int64_t* cols, int64_t n_out,
                               void* out, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(hist && out, "bs_delay_gather: NULL pointer");
  BS_CHECK_ARG(length > 0 && slot_elems >= 0 && n_out >= 0, "bs_delay_gather: bad sizes");
  BS_CHECK_ARG(cols != nullptr || n_out <= slot_elems,
               "bs_delay_gather: %lld outputs from a slot of %lld without column indices",
               (long long)n_out, (long long)slot_elems);
  if (n_out == 0) return BS_OK;
  hipStream_t s = bs_stream(stream);
  const int g = grid_for(n_out);
  switch (elem_bytes) {
    case 1:
      k_gather<uint8_t><<<g, kBlock, 0, s>>>((const uint8_t*)hist, length, slot_elems, cur, step,
                                             steps, cols, n_out, (uint8_t*)out);
      break;
    case 2:
      k_gather<uint16_t><<<g, kBlock, 0, s>>>((const uint16_t*)hist, length, slot_elems, cur,
                                              step, steps, cols, n_out, (uint16_t*)out);
      break;
    case 4:
      k_gather<uint32_t><<<g, kBlock, 0, s>>>((const uint32_t*)hist, length, slot_elems, cur,
                                              step, steps, cols, n_out, (uint32_t*)out);
      break;
    case 8:
      k_gather<uint64_t><<<g, kBlock, 0, s>>>((const uint64_t*)hist, length, slot_elems, cur,
                                              step, steps, cols, n_out, (uint64_t*)out);
      break;
    default:
      bs_set_error("bs_delay_gather: element size %d not in {1, 2, 4, 8}", elem_bytes);
      return BS_ERR_INVALID;
  }
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_delay_taps_f32(const float* hist, int32_t length, int64_t slot_elems,
                                 int32_t taps, const int32_t* slots, const float* weights,
                                 const int64_t* cols, int64_t n_out, float* out,
                                 bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(hist && out && slots && weights, "bs_delay_taps_f32: NULL pointer");
  BS_CHECK_ARG(taps >= 1 && taps <= kMaxTaps, "bs_delay_taps_f32: %d taps not in [1, %d]", taps,
               kMaxTaps);
  BS_CHECK_ARG(length > 0 && slot_elems >= 0 && n_out >= 0, "bs_delay_taps_f32: bad sizes");
  BS_CHECK_ARG(cols != nullptr || n_out <= slot_elems,
               "bs_delay_taps_f32: %lld outputs from a slot of %lld without column indices",
               (long long)n_out, (long long)slot_elems);
  Taps tp;
  tp.n = taps;
  for (int q = 0; q < kMaxTaps; ++q) {
    tp.slot[q] = q < taps ? slots[q] : 0;
    tp.w[q] = q < taps ? weights[q] : 0.0f;
    BS_CHECK_ARG(tp.slot[q] >= 0 && tp.slot[q] < length, "bs_delay_taps_f32: slot %d outside [0, %d)",
                 tp.slot[q], length);
  }
  if (n_out == 0) return BS_OK;
  k_taps<<<grid_for(n_out), kBlock, 0, bs_stream(stream)>>>(hist, slot_elems, tp, cols, n_out,
                                                            out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

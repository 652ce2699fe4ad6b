// Shared host/device helpers for the brainstate_amd HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/brainstate_amd.h"

// ---------------------------------------------------------------- errors
// Thread-local message for bs_last_error(); every entry point returns a status.
void bs_set_error(const char* fmt, ...);
void bs_clear_error();

#define BS_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      bs_set_error(__VA_ARGS__);         \
      return BS_ERR_INVALID;             \
    }                                    \
  } while (0)

#define BS_CHECK_HIP(expr)                                                    \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess) {                                                   \
      bs_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),     \
                   __FILE__, __LINE__);                                       \
      return BS_ERR_LAUNCH;                                                   \
    }                                                                         \
  } while (0)

#define BS_CHECK_LAUNCH()                                                     \
  do {                                                                        \
    hipError_t e_ = hipGetLastError();                                        \
    if (e_ != hipSuccess) {                                                   \
      bs_set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(e_), \
                   __FILE__, __LINE__);                                       \
      return BS_ERR_LAUNCH;                                                   \
    }                                                                         \
  } while (0)

static inline hipStream_t bs_stream(bs_stream_t s) { return (hipStream_t)s; }

// Number of compute units of the current device (cached per device).
int bs_num_cus();

// ---------------------------------------------------------------- device helpers
#define BS_WAVE 64

__device__ __forceinline__ int bs_lane() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// Number of set bits of a 64-bit wave mask in lanes below this lane.
__device__ __forceinline__ int bs_rank_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint64_t bs_ballot(bool p) {
  return __ballot(p);
}

// Hardware fp32 add at the target address; the result is not returned.
__device__ __forceinline__ void bs_atomic_add_f32(float* p, float v) {
  unsafeAtomicAdd(p, v);
}

// Murmur3 32-bit finaliser; spike-set digests are sums of mix32(i) mod 2^32.
__host__ __device__ __forceinline__ uint32_t bs_mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  x ^= x >> 16;
  return x;
}

// ---------------------------------------------------------------- ordered block compaction
// Workspace layout for ordered (ascending) stream compaction with decoupled look-back
// (Merrill & Garland, "Single-pass Parallel Prefix Scan with Decoupled Look-back", 2016).
// Blocks take tickets in launch order, so a block only ever waits for blocks that
// already hold a ticket, i.e. that are resident and running: every wait ends.
// The block with the last ticket resets the ticket and advances the epoch once its
// look-back is done, so the workspace needs one zero-fill when allocated and never again.
struct bs_scan_ws {
  uint32_t ticket;
  uint32_t done;      // unused (kept for the layout)
  uint32_t epoch;     // starts at 0, stays below 2^32 - 1; status words carry (epoch+1)
  uint32_t pad[61];   // status words start at 256 B
  // uint64_t status[nblocks] follows
};

#define BS_SCAN_WS_HEADER 256
#define BS_ST_AGG 1u
#define BS_ST_INC 2u

__device__ __forceinline__ uint64_t* bs_scan_status(bs_scan_ws* ws) {
  return (uint64_t*)((char*)ws + BS_SCAN_WS_HEADER);
}
int bs_fill_f32(float* p, int64_t n, float v, hipStream_t s);

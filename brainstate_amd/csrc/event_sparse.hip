// N2a / N2b: event-driven sparse mat-vec for fixed-num and CSR connectivity.
//
// Scatter (pre-major): waves stride over (active row, 64-synapse chunk) work items; each
// lane loads one target index and weight (a row's synapses are contiguous, so a wave
// reads 256 B of indices and 256 B of weights per chunk) and issues one hardware fp32
// atomic add.  The number of active rows is read on the device, so the launch needs
// no host synchronisation.
//
// Gather (post-major, SELL-64x4): one wave per slice of 64 posts, lane = post.  Each step
// loads the lane's next 4 columns of pre indices as one 16-byte word (1 KB per wave), tests
// the spike of each and adds the weight in column order, so every post accumulates its
// incoming synapses in ascending (pre, k) order -- bit-identical to a sequential pre-major
// scatter, with no atomics.
#include "common.h"

namespace {

constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void k_fill_f32(float* __restrict__ p, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock)
    p[i] = v;
}

template <bool kCsr, bool kHet>
__global__ __launch_bounds__(kBlock) void k_scatter(const int32_t* __restrict__ active,
                                                    const int32_t* __restrict__ n_active_p,
                                                    int32_t n_pre,
                                                    const int32_t* __restrict__ indptr,
                                                    const int32_t* __restrict__ indices,
                                                    int32_t k, const float* __restrict__ w,
                                                    float w_homo, int32_t n_post,
                                                    float* __restrict__ out) {
  int32_t na = *n_active_p;
  na = na < 0 ? 0 : (na > n_pre ? n_pre : na);
  const int lane = bs_lane();
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE;
  const int64_t nwaves = (int64_t)gridDim.x * (kBlock / BS_WAVE);
  if (!kCsr) {
    const int32_t cpr = (k + BS_WAVE - 1) / BS_WAVE;  // 64-synapse chunks per row
    const int64_t items = (int64_t)na * cpr;
    for (int64_t it = wave; it < items; it += nwaves) {
      const int32_t a = (int32_t)(it / cpr);
      const int32_t c = (int32_t)(it - (int64_t)a * cpr);
      const int32_t row = active[a];
      const int32_t t = c * BS_WAVE + lane;
      if ((uint32_t)row < (uint32_t)n_pre && t < k) {
        const int64_t s = (int64_t)row * k + t;
        const int32_t j = indices[s];
        const float v = kHet ? w[s] : w_homo;
        if ((uint32_t)j < (uint32_t)n_post) bs_atomic_add_f32(out + j, v);
      }
    }
  } else {
    const int32_t nnz = indptr[n_pre];
    for (int64_t a = wave; a < na; a += nwaves) {
      const int32_t row = active[a];
      if ((uint32_t)row >= (uint32_t)n_pre) continue;
      int32_t beg = indptr[row], end = indptr[row + 1];
      beg = beg < 0 ? 0 : beg;
      end = end > nnz ? nnz : end;
      for (int32_t s = beg + lane; s < end; s += BS_WAVE) {
        const int32_t j = indices[s];
        const float v = kHet ? w[s] : w_homo;
        if ((uint32_t)j < (uint32_t)n_post) bs_atomic_add_f32(out + j, v);
      }
    }
  }
}

// Spikes -> bitmap, one ballot per 64 spikes: bits[w] bit l <=> spk[32*w + l] != 0.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_pack(const T* __restrict__ spk, int32_t n,
                                                 uint32_t* __restrict__ bits) {
  const int lane = bs_lane();
  const int64_t nwords = ((int64_t)n + 31) / 32;
  for (int64_t base = ((int64_t)blockIdx.x * kBlock + threadIdx.x) - lane;
       base < (int64_t)n; base += (int64_t)gridDim.x * kBlock) {
    const int64_t i = base + lane;
    const bool a = i < n && spk[i] != T(0);
    const uint64_t m = bs_ballot(a);
    const int64_t w = base / 32;
    if (lane == 0 && w < nwords) bits[w] = (uint32_t)m;
    if (lane == 1 && w + 1 < nwords) bits[w + 1] = (uint32_t)(m >> 32);
  }
}

// Gather over SELL-64x4: wave = slice of 64 posts, lane = post; kU 16-byte groups of 4 pre
// indices in flight per lane; the spike test reads a bitmap held in LDS (kLds) or global
// memory.
template <bool kHet, bool kLds>
__global__ __launch_bounds__(kBlock) void k_gather(const uint32_t* __restrict__ bits,
                                                   int32_t n_pre,
                                                   const int64_t* __restrict__ slice_ptr,
                                                   const int32_t* __restrict__ sell_pre,
                                                   const float* __restrict__ sell_w,
                                                   float w_homo, int32_t n_post,
                                                   float* __restrict__ out) {
  constexpr int kGU = 8;  // 16-byte index groups per stage (16: slower, 2x the registers)
  extern __shared__ uint32_t s_bits[];
  const int32_t nwords = (n_pre + 31) / 32;
  if (kLds) {
    for (int32_t w = threadIdx.x; w < nwords; w += kBlock) s_bits[w] = bits[w];
    __syncthreads();
  }
  const uint32_t* bm = kLds ? s_bits : bits;
  const int lane = bs_lane();
  const int64_t slice = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE;
  const int64_t n_slices = ((int64_t)n_post + BS_WAVE - 1) / BS_WAVE;
  if (slice >= n_slices) return;
  const int64_t beg = slice_ptr[slice];
  const int64_t ngrp = (slice_ptr[slice + 1] - beg) / (4 * BS_WAVE);  // groups of 4 columns
  const int4* pre4 = (const int4*)(sell_pre + beg) + lane;
  float acc = 0.0f;
  const auto on = [&](int32_t i) {
    return (uint32_t)i < (uint32_t)n_pre && ((bm[i >> 5] >> (i & 31)) & 1u);
  };
  const float4* w4 = kHet ? (const float4*)(sell_w + beg) + lane : nullptr;
  int64_t g = 0;
  // two stages of kGU 16-byte index groups: the next stage's indices are loaded before this
  // stage's spike lookups, weight loads and adds, which stay in column order (100k x 100k,
  // K = 1000: 121 / 146 / 165 -> 112 / 125 / 158 us at p = 0.001 / 0.01 / 0.1; a third stage
  // for the weights, loaded one block ahead of their adds, measured slower)
  auto ld = [&](int64_t g0, int4 (&q)[kGU]) {
#pragma unroll
    for (int u = 0; u < kGU; ++u) q[u] = pre4[(g0 + u) * BS_WAVE];
  };
  auto use = [&](int64_t g0, const int4 (&q)[kGU]) {
    uint32_t act[kGU];  // bit e: column 4(g0+u)+e is an active synapse
    float4 wq[kGU];
#pragma unroll
    for (int u = 0; u < kGU; ++u) {
      act[u] = (uint32_t)on(q[u].x) | ((uint32_t)on(q[u].y) << 1) | ((uint32_t)on(q[u].z) << 2) |
               ((uint32_t)on(q[u].w) << 3);
      wq[u] = make_float4(w_homo, w_homo, w_homo, w_homo);
      if (kHet && act[u]) wq[u] = w4[(g0 + u) * BS_WAVE];  // this lane's 4 weights, one load
    }
#pragma unroll
    for (int u = 0; u < kGU; ++u) {
      if (act[u] & 1u) acc += wq[u].x;
      if (act[u] & 2u) acc += wq[u].y;
      if (act[u] & 4u) acc += wq[u].z;
      if (act[u] & 8u) acc += wq[u].w;
    }
  };
  if (kGU <= ngrp) {
    int4 qa[kGU], qb[kGU];
    ld(0, qa);
    for (; g + 2 * kGU <= ngrp; g += 2 * kGU) {
      __builtin_amdgcn_sched_barrier(0);
      ld(g + kGU, qb);
      __builtin_amdgcn_sched_barrier(0);
      use(g, qa);
      if (g + 3 * kGU <= ngrp) {
        __builtin_amdgcn_sched_barrier(0);
        ld(g + 2 * kGU, qa);
        __builtin_amdgcn_sched_barrier(0);
      }
      use(g + kGU, qb);
    }
    if (g + kGU <= ngrp) {  // qa holds stage g (loaded above, or before the loop)
      use(g, qa);
      g += kGU;
    }
  }
  for (; g < ngrp; ++g) {
    const int4 q = pre4[g * BS_WAVE];
    const int32_t iv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (on(iv[e])) acc += kHet ? sell_w[beg + (g * BS_WAVE + lane) * 4 + e] : w_homo;
  }
  const int64_t j = slice * BS_WAVE + lane;
  if (j < n_post) out[j] = acc;
}

// Fused event mat-vec straight from the spike vector: workgroup w owns pre rows
// [w*rows, (w+1)*rows); it compacts its active rows into LDS (wave ballots), then adds the
// synapses of those rows.  If the whole output fits in LDS (n_post <= kLdsPosts) and the
// workgroup has at least kLdsRatio events per output, the events of per-synapse weights are
// first aggregated with LDS atomics and each touched output receives one global atomic;
// otherwise every event is one global atomic.  The choice is made per workgroup from its own
// event count.
constexpr int kLdsPosts = 16384;
constexpr int kLdsRatio = 4;
constexpr int kRowsCap = 1024;

// kVal: each event is weighted by its spike value (sum_i x[i] * w[i,k]); otherwise by 1.
// Batched: blockIdx.y selects the batch row (spike row b at spk + b * n_pre, output row at
// out + b * n_post); the connectivity is shared by every row.
template <typename T, bool kCsr, bool kHet, bool kVal = false>
__global__ __launch_bounds__(kBlock) void k_matvec(const T* __restrict__ spk, int32_t n_pre,
                                                   int32_t rows, const int32_t* __restrict__ indptr,
                                                   const int32_t* __restrict__ indices, int32_t k,
                                                   const float* __restrict__ w, float w_homo,
                                                   int32_t n_post, float* __restrict__ out) {
  spk += (int64_t)blockIdx.y * n_pre;
  out += (int64_t)blockIdx.y * n_post;
  __shared__ int32_t s_rows[kRowsCap];
  __shared__ int32_t s_wave[kBlock / BS_WAVE];
  __shared__ int32_t s_nev;
  extern __shared__ float s_acc[];
  const int lane = bs_lane();
  const int wid = threadIdx.x / BS_WAVE;
  const int64_t r0 = (int64_t)blockIdx.x * rows;
  int32_t count = 0;
  for (int32_t off = 0; off < rows; off += kBlock) {
    const int64_t r = r0 + off + threadIdx.x;
    const bool a = off + (int32_t)threadIdx.x < rows && r < n_pre && spk[r] != T(0);
    const uint64_t m = bs_ballot(a);
    if (lane == 0) s_wave[wid] = __popcll(m);
    __syncthreads();
    int32_t pos = count, tot = 0;
#pragma unroll
    for (int v = 0; v < kBlock / BS_WAVE; ++v) {
      pos += v < wid ? s_wave[v] : 0;
      tot += s_wave[v];
    }
    if (a) s_rows[pos + bs_rank_below(m)] = (int32_t)r;
    count += tot;
    __syncthreads();
  }
  if (count == 0) return;
  // events of this workgroup
  if (threadIdx.x == 0) {
    int64_t ev = 0;
    if (!kCsr) {
      ev = (int64_t)count * k;
    } else {
      for (int32_t i = 0; i < count; ++i) ev += indptr[s_rows[i] + 1] - indptr[s_rows[i]];
    }
    s_nev = ev > 0x7FFFFFFF ? 0x7FFFFFFF : (int32_t)ev;
  }
  __syncthreads();
  // Homogeneous weights always go direct: sums of one repeated value are order-free and exact
  // only as a single chain of +w, which LDS partial sums would break.
  const bool use_lds =
      (kHet || kVal) && n_post <= kLdsPosts && (int64_t)s_nev >= (int64_t)kLdsRatio * n_post;
  if (use_lds) {
    for (int32_t j = threadIdx.x; j < n_post; j += kBlock) s_acc[j] = 0.0f;
    __syncthreads();
  }
  const int32_t nnz = kCsr ? indptr[n_pre] : 0;
  for (int32_t a = wid; a < count; a += kBlock / BS_WAVE) {  // one wave per active row
    const int32_t row = s_rows[a];
    const float xv = kVal ? (float)spk[row] : 1.0f;
    int64_t beg, end;
    if (kCsr) {
      beg = indptr[row];
      end = indptr[row + 1];
      beg = beg < 0 ? 0 : beg;
      end = end > nnz ? nnz : end;
    } else {
      beg = (int64_t)row * k;
      end = beg + k;
    }
    for (int64_t s = beg + lane; s < end; s += BS_WAVE) {
      const int32_t j = indices[s];
      const float v = kVal ? (kHet ? w[s] : w_homo) * xv : (kHet ? w[s] : w_homo);
      if ((uint32_t)j < (uint32_t)n_post) {
        if (use_lds) atomicAdd(&s_acc[j], v);
        else bs_atomic_add_f32(out + j, v);
      }
    }
  }
  if (use_lds) {
    __syncthreads();
    for (int32_t j = threadIdx.x; j < n_post; j += kBlock) {
      const float v = s_acc[j];
      if (v != 0.0f) bs_atomic_add_f32(out + j, v);
    }
  }
}

constexpr int kVjpU = 8;  // 64-synapse chunks per wave and round in k_matvec_vjp

// Reverse mode of the event mat-vec y[j] = sum_{i,k: idx[i,k]=j} x[i] * w[i,k] (x = spike
// value; 1 for byte spikes): one wave per pre row i gathers g[idx[i,k]] over the row and
//   grad_x[i]   = sum_k w[i,k] * g[idx[i,k]]            (lane partials, then a wave sum)
//   grad_w[i,k] = x[i] * g[idx[i,k]]                    (per-synapse weights)
//   grad_w[0]  += x[i] * sum_k g[idx[i,k]]              (homogeneous weight; one atomic/row)
// Synapses with out-of-range targets contribute nothing, as in the forward pass.
template <typename T, bool kCsr, bool kHet>
__global__ __launch_bounds__(kBlock) void k_matvec_vjp(const T* __restrict__ spk, int32_t n_pre,
                                                       const int32_t* __restrict__ indptr,
                                                       const int32_t* __restrict__ indices,
                                                       int32_t k, const float* __restrict__ w,
                                                       float w_homo, int32_t n_post,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ gx,
                                                       float* __restrict__ gw) {
  const int lane = bs_lane();
  const int64_t nw = (int64_t)gridDim.x * (kBlock / BS_WAVE);
  const int32_t nnz = kCsr ? indptr[n_pre] : 0;
  for (int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE; row < n_pre;
       row += nw) {
    int64_t beg, end;
    if (kCsr) {
      beg = indptr[row];
      end = indptr[row + 1];
      beg = beg < 0 ? 0 : beg;
      end = end > nnz ? nnz : end;
    } else {
      beg = row * k;
      end = beg + k;
    }
    const float xv = (float)spk[row];
    float sx = 0.0f, sg = 0.0f;
    // kVjpU chunks of 64 synapses per round, every index, weight and gathered g of the round
    // loaded before any is added (one dependent pair of round trips per round instead of one
    // per chunk); each lane still adds its synapses in ascending order (100k x 100k, K = 1000:
    // 774 -> 712 us; what remains is ~1e8 random 4-byte gathers of g from L2 per call)
    for (int64_t s0 = beg + lane; s0 < end; s0 += BS_WAVE * kVjpU) {
      int32_t jj[kVjpU];
      float wv[kVjpU], gj[kVjpU];
#pragma unroll
      for (int u = 0; u < kVjpU; ++u) {
        const int64_t s = s0 + (int64_t)u * BS_WAVE;
        jj[u] = s < end ? indices[s] : -1;
        wv[u] = kHet && gx && s < end ? w[s] : w_homo;
      }
#pragma unroll
      for (int u = 0; u < kVjpU; ++u) gj[u] = (uint32_t)jj[u] < (uint32_t)n_post ? g[jj[u]] : 0.0f;
#pragma unroll
      for (int u = 0; u < kVjpU; ++u) {
        const int64_t s = s0 + (int64_t)u * BS_WAVE;
        if (s < end) {
          if (gx) sx += wv[u] * gj[u];
          if (kHet && gw) gw[s] = xv * gj[u];
          sg += gj[u];
        }
      }
    }
#pragma unroll
    for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
      sx += __shfl_xor(sx, o);
      sg += __shfl_xor(sg, o);
    }
    if (lane == 0) {
      if (gx) gx[row] = sx;
      if (!kHet && gw && xv != 0.0f) bs_atomic_add_f32(gw, xv * sg);
    }
  }
}

// The same gradients for B batch rows in one launch (spk [B, n_pre], g [B, n_post]): one wave
// per pre row i, the row's synapses read once per batch row (from cache after the first):
//   grad_x[b, i] as k_matvec_vjp forms it for row b (lane partials, then a wave sum);
//   grad_w[i, k] = sum_b x[b, i] * g[b, idx[i, k]], the products added in b order, as adding
//   the per-row gradients one after another does (fp32, no contraction);
//   homogeneous: grad_w[0] += x[b, i] * sum_k g[b, idx[i, k]] per (row, b), one atomic each.
template <typename T, bool kCsr, bool kHet>
__global__ __launch_bounds__(kBlock) void k_matvec_vjp_batch(
    const T* __restrict__ spk, int32_t batch, int32_t n_pre, const int32_t* __restrict__ indptr,
    const int32_t* __restrict__ indices, int32_t k, const float* __restrict__ w, float w_homo,
    int32_t n_post, const float* __restrict__ g, float* __restrict__ gx,
    float* __restrict__ gw) {
  const int lane = bs_lane();
  const int64_t nw = (int64_t)gridDim.x * (kBlock / BS_WAVE);
  const int32_t nnz = kCsr ? indptr[n_pre] : 0;
  for (int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / BS_WAVE; row < n_pre;
       row += nw) {
    int64_t beg, end;
    if (kCsr) {
      beg = indptr[row];
      end = indptr[row + 1];
      beg = beg < 0 ? 0 : beg;
      end = end > nnz ? nnz : end;
    } else {
      beg = row * k;
      end = beg + k;
    }
    for (int32_t b = 0; b < batch; ++b) {
      const float xv = (float)spk[(int64_t)b * n_pre + row];
      const float* gb = g + (int64_t)b * n_post;
      float sx = 0.0f, sg = 0.0f;
      for (int64_t s = beg + lane; s < end; s += BS_WAVE) {
        const int32_t j = indices[s];
        const float gj = (uint32_t)j < (uint32_t)n_post ? gb[j] : 0.0f;
        if (gx) sx += (kHet ? w[s] : w_homo) * gj;
        sg += gj;
      }
#pragma unroll
      for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
        sx += __shfl_xor(sx, o);
        sg += __shfl_xor(sg, o);
      }
      if (lane == 0) {
        if (gx) gx[(int64_t)b * n_pre + row] = sx;
        if (!kHet && gw && xv != 0.0f) bs_atomic_add_f32(gw, xv * sg);
      }
    }
    if (kHet && gw) {
      for (int64_t s = beg + lane; s < end; s += BS_WAVE) {
        const int32_t j = indices[s];
        float acc = 0.0f;
        for (int32_t b = 0; b < batch; ++b) {
          const float gj = (uint32_t)j < (uint32_t)n_post ? g[(int64_t)b * n_post + j] : 0.0f;
          const float prod = (float)spk[(int64_t)b * n_pre + row] * gj;
          acc = acc + prod;
        }
        gw[s] = acc;
      }
    }
  }
}

int grid_for(int64_t work_items_waves) {
  const int64_t cap = (int64_t)bs_num_cus() * 16;
  int64_t b = (work_items_waves + (kBlock / BS_WAVE) - 1) / (kBlock / BS_WAVE);
  if (b < 1) b = 1;
  if (b > cap) b = cap;
  return (int)b;
}

}  // namespace

int bs_fill_f32(float* p, int64_t n, float v, hipStream_t s) {
  if (n <= 0) return BS_OK;
  int64_t b = (n + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)bs_num_cus() * 8;
  if (b > cap) b = cap;
  k_fill_f32<<<(int)b, kBlock, 0, s>>>(p, n, v);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_event_scatter_f32(const int32_t* active, const int32_t* n_active, int32_t n_pre,
                                    const int32_t* indptr, const int32_t* indices, int32_t k,
                                    const float* w, float w_homo, int32_t n_post, float* out,
                                    int32_t accumulate, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_pre >= 0 && n_post >= 0, "bs_event_scatter_f32: negative size");
  BS_CHECK_ARG(indptr != nullptr || k >= 0, "bs_event_scatter_f32: k=%d < 0", k);
  hipStream_t s = bs_stream(stream);
  if (n_post > 0) BS_CHECK_ARG(out != nullptr, "bs_event_scatter_f32: out is NULL");
  if (!accumulate) {
    int rc = bs_fill_f32(out, n_post, 0.0f, s);
    if (rc) return rc;
  }
  if (n_pre == 0 || n_post == 0 || (indptr == nullptr && k == 0)) return BS_OK;
  BS_CHECK_ARG(active && n_active && indices, "bs_event_scatter_f32: NULL pointer");
  const bool het = w != nullptr;
  if (indptr == nullptr) {
    const int64_t cpr = ((int64_t)k + BS_WAVE - 1) / BS_WAVE;
    const int g = grid_for((int64_t)n_pre * cpr);
    if (het)
      k_scatter<false, true><<<g, kBlock, 0, s>>>(active, n_active, n_pre, nullptr, indices, k,
                                                  w, w_homo, n_post, out);
    else
      k_scatter<false, false><<<g, kBlock, 0, s>>>(active, n_active, n_pre, nullptr, indices, k,
                                                   nullptr, w_homo, n_post, out);
  } else {
    const int g = grid_for(n_pre);
    if (het)
      k_scatter<true, true><<<g, kBlock, 0, s>>>(active, n_active, n_pre, indptr, indices, 0, w,
                                                 w_homo, n_post, out);
    else
      k_scatter<true, false><<<g, kBlock, 0, s>>>(active, n_active, n_pre, indptr, indices, 0,
                                                  nullptr, w_homo, n_post, out);
  }
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_spike_pack(const void* spk, int32_t spk_dtype, int32_t n, uint32_t* bits,
                             bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n >= 0, "bs_spike_pack: n=%d < 0", n);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_spike_pack: unknown spike dtype %d", spk_dtype);
  if (n == 0) return BS_OK;
  BS_CHECK_ARG(spk && bits, "bs_spike_pack: NULL pointer");
  hipStream_t s = bs_stream(stream);
  const int g = grid_for(((int64_t)n + BS_WAVE - 1) / BS_WAVE);
  if (spk_dtype == BS_SPK_U8) k_pack<uint8_t><<<g, kBlock, 0, s>>>((const uint8_t*)spk, n, bits);
  else k_pack<float><<<g, kBlock, 0, s>>>((const float*)spk, n, bits);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_event_gather_f32(const uint32_t* spk_bits, int32_t n_pre,
                                   const int64_t* slice_ptr, const int32_t* sell_pre,
                                   const float* sell_w, float w_homo, int32_t n_post, float* out,
                                   bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_pre >= 0 && n_post >= 0, "bs_event_gather_f32: negative size");
  if (n_post == 0) return BS_OK;
  BS_CHECK_ARG(slice_ptr && sell_pre && out && (spk_bits || n_pre == 0),
               "bs_event_gather_f32: NULL pointer");
  BS_CHECK_ARG(((uintptr_t)sell_pre & 15) == 0 && ((uintptr_t)sell_w & 15) == 0,
               "bs_event_gather_f32: sell_pre / sell_w must be 16-byte aligned");
  hipStream_t s = bs_stream(stream);
  const int64_t n_slices = ((int64_t)n_post + BS_WAVE - 1) / BS_WAVE;
  const int g = (int)((n_slices + (kBlock / BS_WAVE) - 1) / (kBlock / BS_WAVE));
  const int64_t nwords = ((int64_t)n_pre + 31) / 32;
  const bool lds = nwords * 4 <= 64 * 1024;
  const size_t shm = lds ? (size_t)nwords * 4 : 0;
  const bool het = sell_w != nullptr;
  if (het && lds)
    k_gather<true, true><<<g, kBlock, shm, s>>>(spk_bits, n_pre, slice_ptr, sell_pre, sell_w,
                                                w_homo, n_post, out);
  else if (het)
    k_gather<true, false><<<g, kBlock, 0, s>>>(spk_bits, n_pre, slice_ptr, sell_pre, sell_w,
                                               w_homo, n_post, out);
  else if (lds)
    k_gather<false, true><<<g, kBlock, shm, s>>>(spk_bits, n_pre, slice_ptr, sell_pre, nullptr,
                                                 w_homo, n_post, out);
  else
    k_gather<false, false><<<g, kBlock, 0, s>>>(spk_bits, n_pre, slice_ptr, sell_pre, nullptr,
                                                w_homo, n_post, out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

namespace {

// Shared launcher of the fused mat-vec (event or value-weighted).
template <bool kVal>
int matvec_launch(const void* spk, int32_t spk_dtype, int32_t batch, int32_t n_pre,
                  const int32_t* indptr, const int32_t* indices, int32_t k, const float* w,
                  float w_homo, int32_t n_post, float* out, int32_t accumulate, hipStream_t s,
                  const char* who) {
  BS_CHECK_ARG(n_pre >= 0 && n_post >= 0, "%s: negative size", who);
  BS_CHECK_ARG(batch >= 1 && batch <= 65535, "%s: batch %d outside [1, 65535]", who, batch);
  BS_CHECK_ARG(indptr != nullptr || k >= 0, "%s: k=%d < 0", who, k);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32, "%s: unknown spike dtype %d",
               who, spk_dtype);
  if (n_post > 0) BS_CHECK_ARG(out != nullptr, "%s: out is NULL", who);
  if (!accumulate) {
    int rc = bs_fill_f32(out, (int64_t)batch * n_post, 0.0f, s);
    if (rc) return rc;
  }
  if (n_pre == 0 || n_post == 0 || (indptr == nullptr && k == 0)) return BS_OK;
  BS_CHECK_ARG(spk && indices, "%s: NULL pointer", who);
  // rows per workgroup: enough workgroups (over all batch rows) to fill the chip, at most
  // kRowsCap rows each
  int64_t g = (int64_t)bs_num_cus() * 4;
  int64_t rows = ((int64_t)n_pre * batch + g - 1) / g;
  if (rows < 64) rows = 64;
  if (rows > kRowsCap) rows = kRowsCap;
  g = ((int64_t)n_pre + rows - 1) / rows;
  const size_t shm = n_post <= kLdsPosts ? (size_t)n_post * sizeof(float) : 0;
  const bool het = w != nullptr, csr = indptr != nullptr;
#define BS_MV(T, C, H)                                                                \
  k_matvec<T, C, H, kVal><<<dim3((unsigned)g, (unsigned)batch), kBlock, shm, s>>>(       \
      (const T*)spk, n_pre, (int32_t)rows, indptr, indices, k, w, w_homo, n_post, out)
  if (spk_dtype == BS_SPK_U8) {
    if (csr) { if (het) BS_MV(uint8_t, true, true); else BS_MV(uint8_t, true, false); }
    else { if (het) BS_MV(uint8_t, false, true); else BS_MV(uint8_t, false, false); }
  } else {
    if (csr) { if (het) BS_MV(float, true, true); else BS_MV(float, true, false); }
    else { if (het) BS_MV(float, false, true); else BS_MV(float, false, false); }
  }
#undef BS_MV
  BS_CHECK_LAUNCH();
  return BS_OK;
}

}  // namespace

extern "C" int bs_event_matvec_f32(const void* spk, int32_t spk_dtype, int32_t n_pre,
                                   const int32_t* indptr, const int32_t* indices, int32_t k,
                                   const float* w, float w_homo, int32_t n_post, float* out,
                                   int32_t accumulate, bs_stream_t stream) {
  bs_clear_error();
  return matvec_launch<false>(spk, spk_dtype, 1, n_pre, indptr, indices, k, w, w_homo, n_post,
                              out, accumulate, bs_stream(stream), "bs_event_matvec_f32");
}

extern "C" int bs_event_matvec_batch_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                         int32_t n_pre, const int32_t* indptr,
                                         const int32_t* indices, int32_t k, const float* w,
                                         float w_homo, int32_t n_post, float* out,
                                         int32_t accumulate, bs_stream_t stream) {
  bs_clear_error();
  return matvec_launch<false>(spk, spk_dtype, batch, n_pre, indptr, indices, k, w, w_homo,
                              n_post, out, accumulate, bs_stream(stream),
                              "bs_event_matvec_batch_f32");
}

extern "C" int bs_value_matvec_f32(const float* x, int32_t n_pre, const int32_t* indptr,
                                   const int32_t* indices, int32_t k, const float* w,
                                   float w_homo, int32_t n_post, float* out, int32_t accumulate,
                                   bs_stream_t stream) {
  bs_clear_error();
  return matvec_launch<true>(x, BS_SPK_F32, 1, n_pre, indptr, indices, k, w, w_homo, n_post,
                             out, accumulate, bs_stream(stream), "bs_value_matvec_f32");
}

extern "C" int bs_value_matvec_batch_f32(const float* x, int32_t batch, int32_t n_pre,
                                         const int32_t* indptr, const int32_t* indices, int32_t k,
                                         const float* w, float w_homo, int32_t n_post,
                                         float* out, int32_t accumulate, bs_stream_t stream) {
  bs_clear_error();
  return matvec_launch<true>(x, BS_SPK_F32, batch, n_pre, indptr, indices, k, w, w_homo, n_post,
                             out, accumulate, bs_stream(stream), "bs_value_matvec_batch_f32");
}

extern "C" int bs_event_matvec_vjp_batch_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                             int32_t n_pre, const int32_t* indptr,
                                             const int32_t* indices, int32_t k, const float* w,
                                             float w_homo, int32_t n_post, const float* grad_out,
                                             float* grad_spk, float* grad_w,
                                             bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(batch >= 0 && n_pre >= 0 && n_post >= 0,
               "bs_event_matvec_vjp_batch_f32: negative size");
  BS_CHECK_ARG(indptr != nullptr || k >= 0, "bs_event_matvec_vjp_batch_f32: k=%d < 0", k);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_event_matvec_vjp_batch_f32: unknown spike dtype %d", spk_dtype);
  hipStream_t s = bs_stream(stream);
  const bool het = w != nullptr, csr = indptr != nullptr;
  if (grad_w && !het) {  // homogeneous: one scalar, accumulated with atomics below
    int rc = bs_fill_f32(grad_w, 1, 0.0f, s);
    if (rc) return rc;
  }
  if (n_pre == 0 || (!grad_spk && !grad_w)) return BS_OK;
  BS_CHECK_ARG(spk && indices && (grad_out || n_post == 0 || batch == 0),
               "bs_event_matvec_vjp_batch_f32: NULL pointer");
  if (!csr && k == 0) {  // no synapse: grad_spk is zero, grad_w empty
    return grad_spk ? bs_fill_f32(grad_spk, (int64_t)batch * n_pre, 0.0f, s) : BS_OK;
  }
  // batch == 0 or n_post == 0 go through the kernel: it writes grad_w = 0 (g never read)
  const int g = grid_for(n_pre);
#define BS_VJPB(T, C, H)                                                                    \
  k_matvec_vjp_batch<T, C, H><<<g, kBlock, 0, s>>>((const T*)spk, batch, n_pre, indptr,       \
                                                   indices, k, w, w_homo, n_post, grad_out,   \
                                                   grad_spk, grad_w)
  if (spk_dtype == BS_SPK_U8) {
    if (csr) { if (het) BS_VJPB(uint8_t, true, true); else BS_VJPB(uint8_t, true, false); }
    else { if (het) BS_VJPB(uint8_t, false, true); else BS_VJPB(uint8_t, false, false); }
  } else {
    if (csr) { if (het) BS_VJPB(float, true, true); else BS_VJPB(float, true, false); }
    else { if (het) BS_VJPB(float, false, true); else BS_VJPB(float, false, false); }
  }
#undef BS_VJPB
  BS_CHECK_LAUNCH();
  return BS_OK;
}

extern "C" int bs_event_matvec_vjp_f32(const void* spk, int32_t spk_dtype, int32_t n_pre,
                                       const int32_t* indptr, const int32_t* indices, int32_t k,
                                       const float* w, float w_homo, int32_t n_post,
                                       const float* grad_out, float* grad_spk, float* grad_w,
                                       bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_pre >= 0 && n_post >= 0, "bs_event_matvec_vjp_f32: negative size");
  BS_CHECK_ARG(indptr != nullptr || k >= 0, "bs_event_matvec_vjp_f32: k=%d < 0", k);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_event_matvec_vjp_f32: unknown spike dtype %d", spk_dtype);
  hipStream_t s = bs_stream(stream);
  const bool het = w != nullptr, csr = indptr != nullptr;
  if (grad_w && !het) {  // homogeneous: one scalar, accumulated with atomics below
    int rc = bs_fill_f32(grad_w, 1, 0.0f, s);
    if (rc) return rc;
  }
  if (n_pre == 0 || (!grad_spk && !grad_w)) return BS_OK;
  BS_CHECK_ARG(spk && indices && (grad_out || n_post == 0),
               "bs_event_matvec_vjp_f32: NULL pointer");
  if (n_post == 0 || (!csr && k == 0)) {  // no synapse: every gradient is zero
    if (grad_spk) {
      int rc = bs_fill_f32(grad_spk, n_pre, 0.0f, s);
      if (rc) return rc;
    }
    return BS_OK;
  }
  const int g = grid_for(n_pre);
#define BS_VJP(T, C, H)                                                                   \
  k_matvec_vjp<T, C, H><<<g, kBlock, 0, s>>>((const T*)spk, n_pre, indptr, indices, k, w, \
                                             w_homo, n_post, grad_out, grad_spk, grad_w)
  if (spk_dtype == BS_SPK_U8) {
    if (csr) { if (het) BS_VJP(uint8_t, true, true); else BS_VJP(uint8_t, true, false); }
    else { if (het) BS_VJP(uint8_t, false, true); else BS_VJP(uint8_t, false, false); }
  } else {
    if (csr) { if (het) BS_VJP(float, true, true); else BS_VJP(float, true, false); }
    else { if (het) BS_VJP(float, false, true); else BS_VJP(float, false, false); }
  }
#undef BS_VJP
  BS_CHECK_LAUNCH();
  return BS_OK;
}

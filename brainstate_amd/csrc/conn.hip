// Connectivity construction on the device (brainstate/nn/_event_fixedprob.py:142-196).
//
// With replacement (allow_multi_conn=True) the reference draws
// numpy.random.RandomState(seed).randint(0, n_post, (n_pre, K)) on the host (:163-168), then,
// for afferent_ratio < 1, rng.random(n_pre) < afferent_ratio from the same stream (:186).
// That stream is reproduced here bit for bit:
//   * MT19937 (Matsumoto & Nishimura 1998) seeded with init_genrand(seed), state regenerated in
//     blocks of 624 words, outputs tempered;
//   * numpy's legacy bounded integers: draw = word & mask with mask the smallest 2^j - 1 >=
//     n_post - 1, redrawn while draw > n_post - 1 (no draw at all when n_post == 1);
//   * random(): (a * 2^26 + b) / 2^53 with a = word >> 5, b = next word >> 6.
// The twist is sequential across blocks but splits into three dependency stages within one
// (i < 227 reads only old words; 227 <= i < 454 reads new words < 227; i >= 454 reads new
// words < 397), so one workgroup runs only the twists (three barriers per block) for a word
// budget of expected draws + 12 standard deviations, and parallel passes temper, count the
// accepted draws per block, scan the counts and place every accepted draw.
//
// Without replacement (allow_multi_conn=False) the reference uses its JAX generator
// (init_indices_without_replace, :39-62), which cannot be reproduced without JAX.  Here each
// row draws K values with Philox4x32-10 (Salmon et al. 2011, counter = (row, position,
// round, attempt), key = seed) and Lemire's unbiased bounded integers, then redraws the later
// copy of every repeated value until the row is duplicate-free; the row keeps draw order.
#include <cmath>

#include "common.h"

namespace {

constexpr int kMtN = 624;
constexpr int kMtM = 397;
constexpr uint32_t kMtA = 0x9908b0dfu;
constexpr int kGen = 256;  // generator workgroup (one wave per quarter of a block)

__device__ __forceinline__ uint32_t mt_mix(uint32_t a, uint32_t b) {
  const uint32_t y = (a & 0x80000000u) | (b & 0x7fffffffu);
  return (y >> 1) ^ ((y & 1u) ? kMtA : 0u);
}

__device__ __forceinline__ uint32_t mt_temper(uint32_t y) {
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

// Rank of word i of a 624-word block among the block's accepted words, given per-(chunk,
// wave) accept counts s_cw[3][4] (words i = 256 * chunk + 64 * wave + lane).
__device__ __forceinline__ uint32_t block_rank(const uint32_t (*s_cw)[4], int chunk, int wave,
                                               uint64_t ballot) {
  uint32_t r = 0;
  for (int c = 0; c < chunk; ++c) r += s_cw[c][0] + s_cw[c][1] + s_cw[c][2] + s_cw[c][3];
  for (int w = 0; w < wave; ++w) r += s_cw[chunk][w];
  return r + (uint32_t)bs_rank_below(ballot);
}

// Sequential part: the twists only.  Writes `blocks` blocks of 624 untempered state words.
__global__ __launch_bounds__(kGen) void k_mt_twist(uint32_t seed, int64_t blocks,
                                                   uint32_t* __restrict__ words) {
  __shared__ uint32_t st[2][kMtN];
  const int tid = threadIdx.x;
  if (tid == 0) {  // init_genrand: inherently sequential, once
    uint32_t x = seed;
    for (int i = 0; i < kMtN; ++i) {
      st[0][i] = x;
      x = 1812433253u * (x ^ (x >> 30)) + (uint32_t)(i + 1);
    }
  }
  __syncthreads();
  int cur = 0;
  for (int64_t b = 0; b < blocks; ++b) {
    const uint32_t* o = st[cur];
    uint32_t* nw = st[cur ^ 1];
    uint32_t* dst = words + b * kMtN;
    if (tid < kMtN - kMtM) {
      const uint32_t v = o[tid + kMtM] ^ mt_mix(o[tid], o[tid + 1]);
      nw[tid] = v;
      dst[tid] = v;
    }
    __syncthreads();
    if (tid < kMtN - kMtM) {
      const int i = tid + (kMtN - kMtM);  // 227 .. 453
      const uint32_t v = nw[i - (kMtN - kMtM)] ^ mt_mix(o[i], o[i + 1]);
      nw[i] = v;
      dst[i] = v;
    }
    __syncthreads();
    if (tid < kMtN - 2 * (kMtN - kMtM)) {  // 454 .. 623
      const int i = tid + 2 * (kMtN - kMtM);
      const uint32_t v = nw[i - (kMtN - kMtM)] ^ mt_mix(o[i], i + 1 < kMtN ? o[i + 1] : nw[0]);
      nw[i] = v;
      dst[i] = v;
    }
    __syncthreads();
    cur ^= 1;
  }
}

// Parallel: temper every word in place and count each block's accepted draws.
__global__ __launch_bounds__(kGen) void k_mt_count(uint32_t* __restrict__ words, int64_t blocks,
                                                   uint32_t rng, uint32_t mask,
                                                   uint32_t* __restrict__ counts) {
  __shared__ uint32_t s_c[4];
  const int tid = threadIdx.x;
  for (int64_t b = blockIdx.x; b < blocks; b += gridDim.x) {
    uint32_t c = 0;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int i = q * kGen + tid;
      bool ok = false;
      if (i < kMtN) {
        const uint32_t w = mt_temper(words[b * kMtN + i]);
        words[b * kMtN + i] = w;
        ok = (w & mask) <= rng;
      }
      c += (uint32_t)__popcll(bs_ballot(ok));
    }
    if (bs_lane() == 0) s_c[tid / BS_WAVE] = c;
    __syncthreads();
    if (tid == 0) counts[b] = s_c[0] + s_c[1] + s_c[2] + s_c[3];
    __syncthreads();
  }
}

// One workgroup: ofs[b] = accepted draws before block b (ofs[blocks] = all); info[0] = blocks,
// info[1] = 0 when nothing is drawn (else k_mt_place records the position), info[2] = all.
__global__ __launch_bounds__(1024) void k_mt_scan(const uint32_t* __restrict__ counts,
                                                  int64_t blocks, int64_t need,
                                                  int64_t* __restrict__ ofs,
                                                  int64_t* __restrict__ info) {
  __shared__ int64_t part[1024];
  const int64_t per = (blocks + 1023) / 1024;
  const int64_t lo = threadIdx.x * per;
  const int64_t hi = lo + per < blocks ? lo + per : blocks;
  int64_t c = 0;
  for (int64_t b = lo; b < hi; ++b) c += counts[b];
  part[threadIdx.x] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t acc = 0;
    for (int t = 0; t < 1024; ++t) {
      const int64_t v = part[t];
      part[t] = acc;
      acc += v;
    }
    ofs[blocks] = acc;
    info[0] = blocks;
    info[1] = need == 0 ? 0 : -1;
    info[2] = acc;
  }
  __syncthreads();
  int64_t acc = part[threadIdx.x];
  for (int64_t b = lo; b < hi; ++b) {
    ofs[b] = acc;
    acc += counts[b];
  }
}

// Places accepted draws: out[ofs[b] + rank] = off + (word & mask) for ranks below `need`; the
// draw of rank need - 1 records the stream position after it in info[1].
__global__ __launch_bounds__(kGen) void k_mt_place(const uint32_t* __restrict__ words,
                                                   const int64_t* __restrict__ ofs,
                                                   int64_t blocks, int64_t need, uint32_t rng,
                                                   uint32_t mask, int32_t off,
                                                   int32_t* __restrict__ out,
                                                   int64_t* __restrict__ info) {
  __shared__ uint32_t s_cw[3][4];
  const int tid = threadIdx.x;
  const int wave = tid / BS_WAVE;
  for (int64_t b = blockIdx.x; b < blocks; b += gridDim.x) {
    const int64_t base = ofs[b];
    if (base >= need) break;  // ofs is non-decreasing
    uint32_t w[3];
    uint64_t bal[3];
    bool ok[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const int i = c * kGen + tid;
      ok[c] = false;
      w[c] = 0;
      if (i < kMtN) {
        w[c] = words[b * kMtN + i];
        ok[c] = (w[c] & mask) <= rng;
      }
      bal[c] = bs_ballot(ok[c]);
      if (bs_lane() == 0) s_cw[c][wave] = (uint32_t)__popcll(bal[c]);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if (ok[c]) {
        const int64_t r = base + block_rank(s_cw, c, wave, bal[c]);
        if (r < need) out[r] = off + (int32_t)(w[c] & mask);
        if (r == need - 1) info[1] = b * kMtN + c * kGen + tid + 1;
      }
    }
    __syncthreads();
  }
}

// sel[i] = random() < ratio for the 2 * n words starting after the last index draw.
__global__ void k_mt_select(const uint32_t* __restrict__ words, const int64_t* __restrict__ info,
                            int64_t n_words, int32_t n, double ratio,
                            uint8_t* __restrict__ sel) {
  const int64_t p = info[1];
  if (p < 0 || p + 2 * (int64_t)n > n_words) return;  // reported by the host check
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t a = words[p + 2 * i] >> 5;
    const uint32_t c = words[p + 2 * i + 1] >> 6;
    const double u = ((double)a * 67108864.0 + (double)c) / 9007199254740992.0;
    sel[i] = u < ratio ? 1 : 0;
  }
}

// indptr[i + 1] = k * (selected rows <= i), one workgroup; rows of selected pre neurons are
// copied to out (when given) at indptr[i].
__global__ __launch_bounds__(1024) void k_sel_indptr(const uint8_t* __restrict__ sel, int32_t n,
                                                     int32_t k, int32_t* __restrict__ indptr) {
  __shared__ int64_t part[1024];
  const int64_t per = ((int64_t)n + 1023) / 1024;
  const int64_t lo = threadIdx.x * per;
  const int64_t hi = lo + per < n ? lo + per : n;
  int64_t c = 0;
  for (int64_t i = lo; i < hi; ++i) c += sel[i] ? 1 : 0;
  part[threadIdx.x] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t s = 0;
    for (int t = 0; t < 1024; ++t) {
      const int64_t v = part[t];
      part[t] = s;
      s += v;
    }
    indptr[0] = 0;
  }
  __syncthreads();
  int64_t s = part[threadIdx.x];
  for (int64_t i = lo; i < hi; ++i) {
    s += sel[i] ? 1 : 0;
    indptr[i + 1] = (int32_t)(s * k);
  }
}

__global__ void k_sel_copy(const int32_t* __restrict__ idx, const uint8_t* __restrict__ sel,
                           const int32_t* __restrict__ indptr, int32_t n, int32_t k,
                           int32_t* __restrict__ out) {
  const int64_t total = (int64_t)n * k;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < total;
       x += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = x / k;
    if (sel[i]) out[indptr[i] + (x - i * k)] = idx[x];
  }
}

__global__ void k_fill_i32(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// ---- Philox4x32-10 ----
struct U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 philox(U4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
    c = U4{(uint32_t)(p1 >> 32) ^ c.y ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c.w ^ k1,
           (uint32_t)p0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// Uniform integer in [0, n) for draw (row, pos, round): Lemire's multiply-shift with exact
// rejection, the four Philox words of attempt a tried in order (each word is rejected with
// probability below 1/2, so 16 attempts fail with probability below 2^-64; the last word is
// then kept).
__device__ uint32_t bounded_draw(uint32_t k0, uint32_t k1, uint32_t row, uint32_t pos,
                                 uint32_t round, uint32_t n) {
  const uint32_t thr = (uint32_t)(-n) % n;  // 2^32 mod n
  uint64_t m = 0;
  for (uint32_t a = 0; a < 16; ++a) {
    const U4 r = philox(U4{row, pos, round, a}, k0, k1);
    const uint32_t v[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      m = (uint64_t)v[q] * n;
      if ((uint32_t)m >= thr) return (uint32_t)(m >> 32);
    }
  }
  return (uint32_t)(m >> 32);
}

constexpr int kUniqMax = 2048;     // K per row for the without-replacement sampler
constexpr int kUniqBlock = 256;
constexpr int kUniqRounds = 1 << 16;  // redraw rounds per row (a bound, never reached for K < n_post / 2)

// One workgroup per row: draw K values, sort (value, position) pairs, redraw every position
// holding a repeat of a value seen at an earlier position, until the row has no repeats.
__global__ __launch_bounds__(kUniqBlock) void k_unique_rows(uint32_t k0, uint32_t k1, int32_t n_pre,
                                                            int32_t k, int32_t n_post,
                                                            int32_t* __restrict__ out) {
  __shared__ uint64_t key[kUniqMax];
  __shared__ uint32_t val[kUniqMax];
  __shared__ uint32_t rnd[kUniqMax];
  __shared__ int s_any;
  int kp = 1;
  while (kp < k) kp <<= 1;
  for (int32_t row = blockIdx.x; row < n_pre; row += gridDim.x) {
    for (int p = threadIdx.x; p < k; p += kUniqBlock) {
      rnd[p] = 0;
      val[p] = bounded_draw(k0, k1, (uint32_t)row, (uint32_t)p, 0u, (uint32_t)n_post);
    }
    for (int round = 0; round < kUniqRounds; ++round) {
      for (int p = threadIdx.x; p < kp; p += kUniqBlock)
        key[p] = p < k ? (((uint64_t)val[p] << 32) | (uint32_t)p) : ~0ull;
      if (threadIdx.x == 0) s_any = 0;
      __syncthreads();
      for (int size = 2; size <= kp; size <<= 1) {  // bitonic sort, ascending
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int p = threadIdx.x; p < kp; p += kUniqBlock) {
            const int q = p ^ stride;
            if (q > p) {
              const bool up = (p & size) == 0;
              const uint64_t a = key[p], c = key[q];
              if ((a > c) == up) {
                key[p] = c;
                key[q] = a;
              }
            }
          }
          __syncthreads();
        }
      }
      for (int s = threadIdx.x + 1; s < k; s += kUniqBlock) {
        if ((key[s] >> 32) == (key[s - 1] >> 32)) {  // a later position repeats a value
          const uint32_t p = (uint32_t)key[s];
          rnd[p] += 1;
          val[p] = bounded_draw(k0, k1, (uint32_t)row, p, rnd[p], (uint32_t)n_post);
          s_any = 1;
        }
      }
      __syncthreads();
      const int any = s_any;
      __syncthreads();
      if (!any) break;
    }
    for (int p = threadIdx.x; p < k; p += kUniqBlock) out[(int64_t)row * k + p] = (int32_t)val[p];
    __syncthreads();
  }
}

uint32_t gen_mask(uint32_t rng) {
  uint32_t m = rng;
  m |= m >> 1;
  m |= m >> 2;
  m |= m >> 4;
  m |= m >> 8;
  m |= m >> 16;
  return m;
}

// Words the generator may need: expected draws + 12 standard deviations + a block of slack.
int64_t word_budget(int64_t need, uint32_t rng, int64_t extra) {
  if (need == 0) return extra + 2 * kMtN;
  const double p = ((double)rng + 1.0) / ((double)gen_mask(rng) + 1.0);
  const double mean = (double)need / p;
  const double sd = std::sqrt((double)need * (1.0 - p)) / p;
  return (int64_t)(mean + 12.0 * sd) + extra + 2 * kMtN;
}

struct MtWs {
  int64_t blocks;
  size_t off_words, off_counts, off_ofs, off_info, bytes;
};

MtWs mt_ws(int64_t need, uint32_t rng, int64_t extra) {
  MtWs w;
  w.blocks = (word_budget(need, rng, extra) + kMtN - 1) / kMtN;
  size_t o = 0;
  w.off_words = o;
  o += ((size_t)w.blocks * kMtN * 4 + 255) & ~(size_t)255;
  w.off_counts = o;
  o += ((size_t)w.blocks * 4 + 255) & ~(size_t)255;
  w.off_ofs = o;
  o += ((size_t)(w.blocks + 1) * 8 + 255) & ~(size_t)255;
  w.off_info = o;
  o += 256;
  w.bytes = o;
  return w;
}

}  // namespace

extern "C" size_t bs_conn_fixed_num_workspace_size(int32_t n_pre, int32_t k, int32_t n_post,
                                                    int32_t with_selection) {
  bs_clear_error();
  if (n_pre < 0 || k < 0 || n_post < 1) {
    bs_set_error("bs_conn_fixed_num_workspace_size: bad sizes n_pre=%d k=%d n_post=%d", n_pre,
                 k, n_post);
    return 0;
  }
  const uint32_t rng = (uint32_t)(n_post - 1);
  const int64_t need = rng == 0 ? 0 : (int64_t)n_pre * k;
  return mt_ws(need, rng, with_selection ? 2 * (int64_t)n_pre : 0).bytes;
}

extern "C" int bs_conn_fixed_num(uint32_t seed, int32_t n_pre, int32_t k, int32_t n_post,
                                 int32_t* indices, double afferent_ratio, uint8_t* selected,
                                 void* workspace, size_t workspace_bytes, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_pre >= 0 && k >= 0 && n_post >= 1, "bs_conn_fixed_num: bad sizes");
  BS_CHECK_ARG(indices || (int64_t)n_pre * k == 0, "bs_conn_fixed_num: indices is NULL");
  BS_CHECK_ARG(workspace, "bs_conn_fixed_num: workspace is NULL");
  const uint32_t rng = (uint32_t)(n_post - 1);
  const uint32_t mask = gen_mask(rng);
  const int64_t total = (int64_t)n_pre * k;
  const int64_t need = rng == 0 ? 0 : total;  // n_post == 1: numpy draws nothing
  const int64_t extra = selected ? 2 * (int64_t)n_pre : 0;
  const MtWs w = mt_ws(need, rng, extra);
  BS_CHECK_ARG(workspace_bytes >= w.bytes, "bs_conn_fixed_num: workspace %zu < %zu bytes",
               workspace_bytes, w.bytes);
  hipStream_t s = bs_stream(stream);
  char* ws = (char*)workspace;
  uint32_t* words = (uint32_t*)(ws + w.off_words);
  uint32_t* counts = (uint32_t*)(ws + w.off_counts);
  int64_t* ofs = (int64_t*)(ws + w.off_ofs);
  int64_t* info = (int64_t*)(ws + w.off_info);
  int grid = bs_num_cus() * 8;
  if ((int64_t)grid > w.blocks) grid = (int)w.blocks;
  k_mt_twist<<<1, kGen, 0, s>>>(seed, w.blocks, words);
  BS_CHECK_LAUNCH();
  k_mt_count<<<grid, kGen, 0, s>>>(words, w.blocks, rng, mask, counts);
  BS_CHECK_LAUNCH();
  k_mt_scan<<<1, 1024, 0, s>>>(counts, w.blocks, need, ofs, info);
  BS_CHECK_LAUNCH();
  if (total > 0) {
    if (need == 0) {  // one target: every index is 0
      k_fill_i32<<<bs_num_cus() * 4, 256, 0, s>>>(indices, total, 0);
    } else {
      k_mt_place<<<grid, kGen, 0, s>>>(words, ofs, w.blocks, need, rng, mask, 0, indices, info);
    }
    BS_CHECK_LAUNCH();
  }
  if (selected && n_pre > 0) {
    k_mt_select<<<(n_pre + 255) / 256 < 4096 ? (n_pre + 255) / 256 : 4096, 256, 0, s>>>(
        words, info, w.blocks * kMtN, n_pre, afferent_ratio, selected);
    BS_CHECK_LAUNCH();
  }
  int64_t hinfo[3];
  BS_CHECK_HIP(hipMemcpyAsync(hinfo, info, sizeof(hinfo), hipMemcpyDeviceToHost, s));
  BS_CHECK_HIP(hipStreamSynchronize(s));
  if (hinfo[1] < 0 || hinfo[1] + extra > w.blocks * kMtN) {
    bs_set_error("bs_conn_fixed_num: word budget of %lld blocks exhausted",
                 (long long)w.blocks);
    return BS_ERR_LAUNCH;
  }
  return BS_OK;
}

extern "C" int bs_csr_from_selected(const int32_t* indices, int32_t n_pre, int32_t k,
                                    const uint8_t* selected, int32_t* indptr, int32_t* out,
                                    bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_pre >= 0 && k >= 0, "bs_csr_from_selected: bad sizes");
  BS_CHECK_ARG(selected && indptr, "bs_csr_from_selected: NULL pointer");
  BS_CHECK_ARG(!out || indices, "bs_csr_from_selected: indices is NULL");
  BS_CHECK_ARG((int64_t)n_pre * k < ((int64_t)1 << 31), "bs_csr_from_selected: %lld synapses "
               "exceed int32 offsets", (long long)n_pre * k);
  hipStream_t s = bs_stream(stream);
  k_sel_indptr<<<1, 1024, 0, s>>>(selected, n_pre, k, indptr);
  BS_CHECK_LAUNCH();
  if (out && (int64_t)n_pre * k > 0) {
    k_sel_copy<<<bs_num_cus() * 8, 256, 0, s>>>(indices, selected, indptr, n_pre, k, out);
    BS_CHECK_LAUNCH();
  }
  return BS_OK;
}

extern "C" int bs_conn_fixed_num_unique(uint64_t seed, int32_t n_pre, int32_t k, int32_t n_post,
                                        int32_t* indices, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_pre >= 0 && k >= 0 && n_post >= 1, "bs_conn_fixed_num_unique: bad sizes");
  BS_CHECK_ARG(k <= n_post, "bs_conn_fixed_num_unique: K=%d distinct targets out of %d", k,
               n_post);
  BS_CHECK_ARG(k <= kUniqMax, "bs_conn_fixed_num_unique: K=%d above %d", k, kUniqMax);
  BS_CHECK_ARG(indices || (int64_t)n_pre * k == 0, "bs_conn_fixed_num_unique: indices is NULL");
  if ((int64_t)n_pre * k == 0) return BS_OK;
  int grid = bs_num_cus() * 8;
  if (grid > n_pre) grid = n_pre;
  k_unique_rows<<<grid, kUniqBlock, 0, bs_stream(stream)>>>(
      (uint32_t)seed, (uint32_t)(seed >> 32), n_pre, k, n_post, indices);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

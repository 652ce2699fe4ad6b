// N2a, destination-bucketed: the event mat-vec of fixed-num / CSR connectivity without global
// atomics and without fp32 atomics.
//
// Why: scattered global fp32 atomics on MI355X sustain ~20 G/s chip-wide, so the pre-major
// scatter of config [2] at p = 0.1 (1e7 events) costs > 500 us, while its compulsory bytes
// (indices + weights of the active rows) take ~10 us at HBM speed.  LDS atomics are cheaper,
// but measured on gfx950 ds_add_f32 sustains only ~0.3 lanes per clock per CU (76 us for the
// p = 0.1 case), while integer LDS atomics run at the speed of plain LDS stores (~30 us).
//
// Layout (built once per connectivity, bs_bucket_build): posts are cut into nb buckets of P
// consecutive posts (P <= kMaxP, the LDS accumulator).  Each pre row keeps its synapses
// contiguous but sorted by bucket (stable: original order inside a bucket), with the target
// stored as a 16-bit offset inside its bucket; seg[i][b] is where row i's bucket-b synapses
// start and seg[i][nb] where its valid synapses end (out-of-range targets follow and are
// never read).  The build also fixes a fixed-point exponent S from max|w| and the synapse
// count so that no sum can exceed 2^60 in units of 2^-S.
//
// Step (bs_event_bucket_f32): workgroup (b, r) owns bucket b and the pre rows of row group r.
// It compacts the active rows of its group into LDS (ballots), loads their bucket-b bounds,
// and accumulates their bucket-b synapses into an LDS copy of the bucket with integer LDS
// atomics: each weight rounded to a multiple of 2^-S and added as a 64-bit integer (event
// counts for a homogeneous weight).  It writes the bucket as partial r; a second kernel adds
// the R partials exactly and rounds once: out = fl32(sum) * 2^-S, whatever the order of the
// atomics (deterministic), within half an fp32 ulp of the exact sum of the rounded weights.
// Homogeneous weights: the exact event count c, then w added c times in one chain, which is
// the sequential scatter's result bit for bit.  Non-finite weights fall back to fp32 LDS
// atomics (unspecified order).  HBM traffic: the active rows' synapses once (E x (2 + 4 het)
// bytes) + R partial rows of n_post x 8 bytes written and read.
#include "common.h"

namespace {

constexpr int kBB = 256;          // build: threads per workgroup (one wave per row)
constexpr int kSB = 1024;         // step: threads per workgroup
constexpr int kMaxP = 12288;      // posts per bucket (96 KiB of 64-bit LDS accumulators)
constexpr int kMaxNb = 1024;      // buckets
// Measured on MI355X at config [2] (100k x 100k, K = 1000, p = 0.1): 9 buckets of 11,112
// posts with 28 row groups 30 us; 16 buckets 34 us; 32 buckets 48 us; 8 rows per wave with one
// pass 53 us; a 512-workgroup target 40 us.  fp32 LDS atomics instead of 64-bit integers:
// 76 us.
constexpr int kRowsPer = 4;       // active rows a wave works on at once
constexpr int kPasses = 2;        // 64-synapse passes per row issued together
constexpr int kSpan = 4096;       // rows compacted per span
constexpr int kTargetWgs = 256;   // step grid the row groups aim for
constexpr int kMinRows = 64;      // rows per row group, at least
constexpr int kMinNb = 8;         // buckets, at least (the grid is nb x row groups)

// ---- layout build: one wave per pre row ----
// s_run[wave][b]: synapses of bucket b placed so far (b = nb: out-of-range targets).
__global__ __launch_bounds__(kBB) void k_bucket_count(int32_t n_pre, const int32_t* indptr,
                                                      const int32_t* indices, int32_t k,
                                                      int32_t n_post, int32_t nb, int32_t P,
                                                      int32_t* seg) {
  extern __shared__ int32_t s_cnt[];  // [waves][nb + 1]
  const int lane = bs_lane();
  const int wl = threadIdx.x / BS_WAVE;
  const int64_t i = ((int64_t)blockIdx.x * kBB + threadIdx.x) / BS_WAVE;
  int32_t* cnt = s_cnt + wl * (nb + 1);
  for (int b = lane; b <= nb; b += BS_WAVE) cnt[b] = 0;
  __syncthreads();
  if (i < n_pre) {
    const int64_t beg = indptr ? indptr[i] : i * (int64_t)k;
    const int64_t end = indptr ? indptr[i + 1] : beg + k;
    for (int64_t s = beg + lane; s < end; s += BS_WAVE) {
      const int32_t t = indices[s];
      const int b = (uint32_t)t < (uint32_t)n_post ? t / P : nb;
      atomicAdd(&cnt[b], 1);
    }
  }
  __syncthreads();
  if (i < n_pre && lane == 0) {
    // seg[i][b] = row start + synapses of buckets < b
    int64_t pos = indptr ? indptr[i] : i * (int64_t)k;
    int32_t* sr = seg + i * (int64_t)(nb + 1);
    for (int b = 0; b <= nb; ++b) {
      sr[b] = (int32_t)pos;
      pos += b < nb ? cnt[b] : 0;
    }
  }
}

__global__ __launch_bounds__(kBB) void k_bucket_place(int32_t n_pre, const int32_t* indptr,
                                                      const int32_t* indices, const float* w,
                                                      int32_t k, int32_t n_post, int32_t nb,
                                                      int32_t P, const int32_t* seg,
                                                      uint16_t* lidx, float* lw,
                                                      uint32_t* wmax) {
  extern __shared__ int32_t s_run[];  // [waves][nb + 1]
  const int lane = bs_lane();
  const int wl = threadIdx.x / BS_WAVE;
  const int64_t i = ((int64_t)blockIdx.x * kBB + threadIdx.x) / BS_WAVE;
  int32_t* run = s_run + wl * (nb + 1);
  if (i >= n_pre) return;  // whole wave; no barrier below
  const int32_t* sr = seg + i * (int64_t)(nb + 1);
  for (int b = lane; b <= nb; b += BS_WAVE) run[b] = b < nb ? sr[b] : sr[nb];
  const int64_t beg = indptr ? indptr[i] : i * (int64_t)k;
  const int64_t end = indptr ? indptr[i + 1] : beg + k;
  // max |w| over the row's valid synapses (the bit pattern of a non-negative float orders like
  // its value; NaN sorts above +inf): lane maxima, a wave maximum, one atomic per row
  uint32_t amax = 0u;
  // 64 synapses at a time; each distinct bucket of the chunk is ranked with one ballot, so
  // synapses keep their original order inside a bucket
  for (int64_t s0 = beg; s0 < end; s0 += BS_WAVE) {
    const int64_t s = s0 + lane;
    const bool live = s < end;
    int32_t t = live ? indices[s] : 0;
    const int b = !live ? -1 : ((uint32_t)t < (uint32_t)n_post ? t / P : nb);
    if (lw && live && b < nb) {
      const uint32_t aw = __float_as_uint(w[s]) & 0x7FFFFFFFu;
      amax = aw > amax ? aw : amax;
    }
    uint64_t left = bs_ballot(live);
    while (left) {
      const int leader = __builtin_ctzll(left);
      const int bl = __builtin_amdgcn_readlane(b, leader);
      const uint64_t m = bs_ballot(b == bl);
      const int32_t base = run[bl];  // wave-uniform LDS read
      if (b == bl) {
        const int32_t pos = base + bs_rank_below(m);
        lidx[pos] = (uint16_t)(bl < nb ? t - bl * P : 0);
        if (lw) lw[pos] = w[s];
      }

      if (lane == leader) run[bl] = base + (int32_t)__popcll(m);
      left &= ~m;
    }
  }
  if (lw) {
    for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
      const uint32_t x = (uint32_t)__shfl_xor((int)amax, o);
      amax = x > amax ? x : amax;
    }
    if (lane == 0 && amax) atomicMax(wmax, amax);
  }
}

__global__ void k_u32_zero(uint32_t* p) { *p = 0u; }

// S = 60 - e_w - e_n with max|w| < 2^e_w and (synapses) <= 2^e_n: no sum of events can reach
// 2^60 units of 2^-S.  -1000 flags a non-finite weight; 0 when every weight is 0.
__global__ void k_bucket_qexp(const uint32_t* wmax, int64_t nnz_fixed, const int32_t* indptr,
                              int32_t n_pre, int32_t* qexp) {
  const uint32_t bits = *wmax;
  if (bits >= 0x7F800000u) { *qexp = -1000; return; }
  if (bits == 0u) { *qexp = 0; return; }
  const int64_t nnz = indptr ? (int64_t)indptr[n_pre] - indptr[0] : nnz_fixed;
  int e_n = 0;
  while (((int64_t)1 << e_n) < nnz) ++e_n;
  const int e_w = ilogbf(__uint_as_float(bits)) + 1;
  *qexp = 60 - e_w - e_n;
}

// ---- step ----
// Phases per span of up to kSpan rows of the workgroup's row group:
//   1. compaction of the span's active rows into s_beg (ballots, ascending);
//   2. every thread loads the bucket-b bounds of some active rows (all in flight) into
//      s_beg / s_len;
//   3. waves take kRowsPer rows at a time and issue the loads of up to kPasses 64-synapse
//      passes of all of them before their LDS atomics.
template <typename T, bool kHet>
__global__ __launch_bounds__(kSB) void k_bucket_scatter(const T* __restrict__ spk, int32_t n_pre,
                                                        int32_t rows, int32_t nb, int32_t P,
                                                        const int32_t* __restrict__ seg,
                                                        const uint16_t* __restrict__ lidx,
                                                        const float* __restrict__ lw,
                                                        const int32_t* __restrict__ qexp,
                                                        int32_t n_post, uint64_t* __restrict__ part) {
  __shared__ uint64_t s_acc[kMaxP];        // fixed-point sums, fp32 sums or event counts
  uint32_t* s_acc32 = (uint32_t*)s_acc;
  __shared__ int32_t s_beg[kSpan];
  __shared__ int32_t s_len[kSpan];
  __shared__ int32_t s_wave[kSB / BS_WAVE];
  const int lane = bs_lane();
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / BS_WAVE));
  const int32_t b = blockIdx.x % nb;
  const int32_t r = blockIdx.x / nb;
  const int32_t p0 = b * P;
  const int32_t pn = n_post - p0 < P ? n_post - p0 : P;  // posts in this bucket
  for (int j = threadIdx.x; j < pn; j += kSB) s_acc[j] = 0ull;
  // fixed point (S >= -999) unless a weight is not finite; scale = 2^S exactly
  const int32_t S = kHet ? __builtin_amdgcn_readfirstlane(*qexp) : 0;
  const bool fixed = kHet && S > -1000;
  const double scale = fixed ? ldexp(1.0, S) : 1.0;
  const int64_t r0 = (int64_t)r * rows;
  const int64_t r1 = r0 + rows < n_pre ? r0 + rows : n_pre;
  const int stride = nb + 1;
  for (int64_t c0 = r0; c0 < r1; c0 += kSpan) {
    // 1. active rows of the span, ascending
    int32_t count = 0;
    for (int32_t o = 0; o < kSpan; o += kSB) {
      const int64_t row = c0 + o + threadIdx.x;
      const bool a = row < r1 && spk[row] != T(0);
      const uint64_t m = bs_ballot(a);
      if (lane == 0) s_wave[wid] = __popcll(m);
      __syncthreads();
      int32_t pos = count, tot = 0;
#pragma unroll
      for (int v = 0; v < kSB / BS_WAVE; ++v) {
        pos += v < wid ? s_wave[v] : 0;
        tot += s_wave[v];
      }
      if (a) s_beg[pos + bs_rank_below(m)] = (int32_t)row;
      count += tot;
      __syncthreads();  // s_wave is rewritten next round
    }
    // 2. bounds of bucket b in each active row
    for (int32_t x = threadIdx.x; x < count; x += kSB) {
      const int32_t* sr = seg + (int64_t)s_beg[x] * stride + b;
      const int32_t lo = sr[0], hi = sr[1];
      s_beg[x] = lo;
      s_len[x] = hi - lo;
    }
    __syncthreads();
    // 3. synapses of kRowsPer rows, up to kPasses x 64 each, loads in flight together
    for (int32_t a0 = wid * kRowsPer; a0 < count; a0 += (kSB / BS_WAVE) * kRowsPer) {
      int32_t beg[kRowsPer], len[kRowsPer];
      int32_t maxlen = 0;
#pragma unroll
      for (int q = 0; q < kRowsPer; ++q) {
        const bool ok = a0 + q < count;
        beg[q] = ok ? s_beg[a0 + q] : 0;
        len[q] = ok ? s_len[a0 + q] : 0;
        maxlen = len[q] > maxlen ? len[q] : maxlen;
      }
      for (int32_t e0 = 0; e0 < maxlen; e0 += kPasses * BS_WAVE) {
        uint16_t t[kPasses][kRowsPer];
        float v[kPasses][kRowsPer];
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
#pragma unroll
          for (int q = 0; q < kRowsPer; ++q) {
            const int32_t e = e0 + u * BS_WAVE + lane;
            t[u][q] = 0xFFFFu;
            v[u][q] = 0.0f;
            if (e < len[q]) {
              t[u][q] = lidx[(int64_t)beg[q] + e];
              if (kHet) v[u][q] = lw[(int64_t)beg[q] + e];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
#pragma unroll
          for (int q = 0; q < kRowsPer; ++q) {
            if (t[u][q] != 0xFFFFu) {
              if (!kHet) {
                atomicAdd(&s_acc32[t[u][q]], 1u);
              } else if (fixed) {
                const int64_t qv = (int64_t)__builtin_rint((double)v[u][q] * scale);
                atomicAdd((unsigned long long*)&s_acc[t[u][q]], (unsigned long long)qv);
              } else {
                atomicAdd((float*)&s_acc32[t[u][q]], v[u][q]);
              }
            }
          }
        }
      }
    }
    __syncthreads();  // s_beg / s_len are rewritten by the next span
  }
  __syncthreads();
  uint64_t* dst = part + (int64_t)r * n_post + p0;
  if (kHet && fixed) {
    for (int j = threadIdx.x; j < pn; j += kSB) dst[j] = s_acc[j];
  } else {
    for (int j = threadIdx.x; j < pn; j += kSB) dst[j] = s_acc32[j];
  }
}

// out[j] = (accumulate ? out[j] : 0) + the bucket sums of j:
//   fixed point: the R partials added exactly (64-bit), then fl32(sum) * 2^-S;
//   homogeneous: the total count c of events, then c additions of w (the sequential chain);
//   fp32 fallback: the R partials added in row-group order.
template <bool kHet>
__global__ __launch_bounds__(256) void k_bucket_reduce(int32_t n_post, int32_t R,
                                                       const uint64_t* __restrict__ part,
                                                       const int32_t* __restrict__ qexp,
                                                       float w_homo, int32_t accumulate,
                                                       float* __restrict__ out) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= n_post) return;
  float acc = accumulate ? out[j] : 0.0f;
  const int32_t S = kHet ? *qexp : 0;
  if (kHet && S > -1000) {
    int64_t q = 0;
    int32_t r = 0;
    for (; r + 8 <= R; r += 8) {
      int64_t x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = (int64_t)part[(int64_t)(r + u) * n_post + j];
#pragma unroll
      for (int u = 0; u < 8; ++u) q += x[u];
    }
    for (; r < R; ++r) q += (int64_t)part[(int64_t)r * n_post + j];
    const float v = ldexpf((float)q, -S);
    acc = accumulate ? acc + v : v;
  } else if (kHet) {
    for (int32_t r = 0; r < R; ++r) acc += __uint_as_float((uint32_t)part[(int64_t)r * n_post + j]);
  } else {
    uint32_t c = 0;
    for (int32_t r = 0; r < R; ++r) c += (uint32_t)part[(int64_t)r * n_post + j];
    for (uint32_t u = 0; u < c; ++u) acc += w_homo;
  }
  out[j] = acc;
}

int32_t row_groups(int32_t n_pre, int32_t nb) {
  int64_t R = kTargetWgs / (nb > 0 ? nb : 1);
  const int64_t rmax = ((int64_t)n_pre + kMinRows - 1) / kMinRows;
  if (R > rmax) R = rmax;
  if (R < 1) R = 1;
  return (int32_t)R;
}

int check_layout(int32_t n_pre, int32_t n_post, int32_t nb, int32_t P, const char* who) {
  BS_CHECK_ARG(n_pre >= 0 && n_post >= 0, "%s: negative size", who);
  BS_CHECK_ARG(nb >= 1 && nb <= kMaxNb, "%s: nb=%d outside [1, %d]", who, nb, kMaxNb);
  BS_CHECK_ARG(P >= 1 && P <= kMaxP, "%s: P=%d outside [1, %d]", who, P, kMaxP);
  BS_CHECK_ARG((int64_t)nb * P >= n_post && (int64_t)(nb - 1) * P < (int64_t)n_post + (n_post == 0),
               "%s: nb=%d buckets of P=%d do not tile n_post=%d", who, nb, P, n_post);
  return BS_OK;
}

}  // namespace

extern "C" int bs_bucket_plan(int32_t n_post, int32_t* P_out) {
  bs_clear_error();
  BS_CHECK_ARG(n_post >= 0, "bs_bucket_plan: negative n_post");
  // at least kMinNb buckets (the step grid is nb x row groups; fewer row groups mean fewer
  // partials to write and add), each at most kMaxP posts
  int64_t nb = ((int64_t)n_post + kMaxP - 1) / kMaxP;
  if (nb < kMinNb) nb = kMinNb;
  if (nb > kMaxNb) {
    bs_set_error("bs_bucket_plan: n_post=%d needs more than %d buckets", n_post, kMaxNb);
    return -1;
  }
  int64_t P = ((int64_t)n_post + nb - 1) / nb;
  if (P < 1) P = 1;
  nb = ((int64_t)n_post + P - 1) / P;
  if (nb < 1) nb = 1;
  if (P_out) *P_out = (int32_t)P;
  return (int32_t)nb;
}

extern "C" int bs_bucket_build(int32_t n_pre, const int32_t* indptr, const int32_t* indices,
                               int32_t k, const float* w, int32_t n_post, int32_t nb, int32_t P,
                               int32_t* seg, uint16_t* lidx, float* lw, int32_t* qexp,
                               void* workspace, bs_stream_t stream) {
  bs_clear_error();
  int rc = check_layout(n_pre, n_post, nb, P, "bs_bucket_build");
  if (rc) return rc;
  BS_CHECK_ARG(indptr != nullptr || k >= 0, "bs_bucket_build: k=%d < 0", k);
  BS_CHECK_ARG((w == nullptr) == (lw == nullptr),
               "bs_bucket_build: w and lw must both be given or both be NULL");
  BS_CHECK_ARG(w == nullptr || (qexp != nullptr && workspace != nullptr),
               "bs_bucket_build: per-synapse weights need qexp and a 4-byte workspace");
  if (n_pre == 0) return BS_OK;
  BS_CHECK_ARG(seg != nullptr, "bs_bucket_build: seg is NULL");
  const bool any = indptr != nullptr || k > 0;
  if (any) BS_CHECK_ARG(indices && lidx, "bs_bucket_build: NULL pointer");
  hipStream_t s = bs_stream(stream);
  const int64_t g = ((int64_t)n_pre * BS_WAVE + kBB - 1) / kBB;
  const size_t shm = (size_t)(kBB / BS_WAVE) * (nb + 1) * sizeof(int32_t);
  k_bucket_count<<<(int)g, kBB, shm, s>>>(n_pre, indptr, any ? indices : nullptr, k, n_post, nb,
                                          P, seg);
  BS_CHECK_LAUNCH();
  if (!any) {
    if (w) {
      k_u32_zero<<<1, 1, 0, s>>>((uint32_t*)workspace);
      BS_CHECK_LAUNCH();
      k_bucket_qexp<<<1, 1, 0, s>>>((uint32_t*)workspace, 0, nullptr, n_pre, qexp);
      BS_CHECK_LAUNCH();
    }
    return BS_OK;
  }
  uint32_t* wmax = (uint32_t*)workspace;
  if (w) {
    k_u32_zero<<<1, 1, 0, s>>>(wmax);
    BS_CHECK_LAUNCH();
  }
  k_bucket_place<<<(int)g, kBB, shm, s>>>(n_pre, indptr, indices, w, k, n_post, nb, P, seg, lidx,
                                          lw, w ? wmax : nullptr);
  BS_CHECK_LAUNCH();
  if (w) {
    k_bucket_qexp<<<1, 1, 0, s>>>(wmax, (int64_t)n_pre * k, indptr, n_pre, qexp);
    BS_CHECK_LAUNCH();
  }
  return BS_OK;
}

extern "C" size_t bs_event_bucket_workspace_size(int32_t n_pre, int32_t n_post, int32_t nb) {
  bs_clear_error();
  if (n_pre <= 0 || n_post <= 0 || nb <= 0) return 0;
  return (size_t)row_groups(n_pre, nb) * n_post * sizeof(uint64_t);
}

extern "C" int bs_event_bucket_f32(const void* spk, int32_t spk_dtype, int32_t n_pre,
                                   int32_t n_post, int32_t nb, int32_t P, const int32_t* seg,
                                   const uint16_t* lidx, const float* lw, const int32_t* qexp,
                                   float w_homo, float* out, int32_t accumulate, void* workspace,
                                   size_t workspace_bytes, bs_stream_t stream) {
  bs_clear_error();
  int rc = check_layout(n_pre, n_post, nb, P, "bs_event_bucket_f32");
  if (rc) return rc;
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "bs_event_bucket_f32: unknown spike dtype %d", spk_dtype);
  if (n_post == 0) return BS_OK;
  BS_CHECK_ARG(out != nullptr, "bs_event_bucket_f32: out is NULL");
  hipStream_t s = bs_stream(stream);
  if (n_pre == 0) return accumulate ? BS_OK : bs_fill_f32(out, n_post, 0.0f, s);
  BS_CHECK_ARG(spk && seg && lidx, "bs_event_bucket_f32: NULL pointer");
  BS_CHECK_ARG(lw == nullptr || qexp != nullptr, "bs_event_bucket_f32: qexp is NULL");
  const int32_t R = row_groups(n_pre, nb);
  const size_t need = (size_t)R * n_post * sizeof(uint64_t);
  BS_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "bs_event_bucket_f32: workspace of %zu bytes needed (got %zu)", need,
               workspace ? workspace_bytes : (size_t)0);
  const int32_t rows = (int32_t)(((int64_t)n_pre + R - 1) / R);
  uint64_t* part = (uint64_t*)workspace;
  const int64_t g = (int64_t)nb * R;
#define BS_BK(T, H)                                                                        \
  k_bucket_scatter<T, H><<<(int)g, kSB, 0, s>>>((const T*)spk, n_pre, rows, nb, P, seg, lidx, \
                                                lw, qexp, n_post, part)
  if (spk_dtype == BS_SPK_U8) { if (lw) BS_BK(uint8_t, true); else BS_BK(uint8_t, false); }
  else { if (lw) BS_BK(float, true); else BS_BK(float, false); }
#undef BS_BK
  BS_CHECK_LAUNCH();
  const int gr = (int)(((int64_t)n_post + 255) / 256);
  if (lw) k_bucket_reduce<true><<<gr, 256, 0, s>>>(n_post, R, part, qexp, w_homo, accumulate, out);
  else k_bucket_reduce<false><<<gr, 256, 0, s>>>(n_post, R, part, qexp, w_homo, accumulate, out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

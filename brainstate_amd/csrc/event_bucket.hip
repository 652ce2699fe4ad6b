// N2a, destination-bucketed: the event mat-vec of fixed-num / CSR connectivity without global
// atomics and without fp32 atomics.
//
// Why: scattered global fp32 atomics on MI355X sustain ~20 G/s chip-wide, so the pre-major
// scatter of a 100k x 100k, K = 1000 mat-vec at p = 0.1 (1e7 events) costs > 500 us, while its compulsory bytes
// (indices + weights of the active rows) take ~10 us at HBM speed.  LDS atomics are cheaper,
// but measured on gfx950 ds_add_f32 sustains only ~0.3 lanes per clock per CU (76 us for the
// p = 0.1 case), while integer LDS atomics run at the speed of plain LDS stores (~30 us).
//
// Layout (built once per connectivity, bs_bucket_build): posts are cut into nb buckets of P
// consecutive posts (P <= kMaxP, the LDS accumulator).  Each pre row keeps its synapses
// contiguous but sorted by bucket (stable: original order inside a bucket), with the target
// stored as a 16-bit offset inside its bucket; seg[i][b] is where row i's bucket-b synapses
// start and seg[i][nb] where its valid synapses end (out-of-range targets follow and are
// never read).  The build also fixes a fixed-point exponent S = min(30 - e_w - e_d, 100) from
// max|w| < 2^e_w and the largest in-degree D <= 2^e_d -- the persistent runner's rule, so an
// E/I step run through this operator adds the same integers as the runner -- : every weight
// rounded to a multiple of 2^-S is an integer below 2^(30 - e_d) in magnitude, formed exactly
// in fp32 (ldexp, round to nearest even, convert), and every output's sum is below 2^30.
//
// Step (bs_event_bucket_f32): workgroup (b, r) owns bucket b and the pre rows of row group r.
// It compacts the active rows of its group into LDS (ballots), loads their bucket-b bounds,
// and accumulates their bucket-b synapses into an LDS copy of the bucket with integer LDS
// atomics: each weight rounded to a multiple of 2^-S and added as a 32-bit integer (event
// counts for a homogeneous weight); every sum of rounded weights stays below 2^31 in
// magnitude, so 32-bit two's complement adds are exact (64-bit accumulators and partials
// before the runner's exponent rule made that bound hold: 100k x 100k, K = 1000, p = 0.1 ... us).  It writes the bucket as partial r; a second kernel adds
// the partials exactly and rounds once: out = fl32(sum) * 2^-S, whatever the order of the
// atomics (deterministic), within half an fp32 ulp of the exact sum of the rounded weights.
// Homogeneous weights: the exact event count c, then w added c times in one chain, which is
// the sequential scatter's result bit for bit.  Non-finite weights fall back to fp32 LDS
// atomics (unspecified order).
//
// The number of row groups follows the spike density, on the device: the grid is launched
// for R groups, every workgroup counts the active rows of the same leading sample of the
// spike vector and derives R_eff <= R (about kActivePer active rows per group); groups
// r >= R_eff exit at once.  With R_eff = 1 the workgroups write `out` themselves and the
// second kernel returns at once, so a sparse step costs one pass over the spikes and the
// active synapses instead of R partial rows written and read.  The single launch (R = 1 on
// the host) skips the estimate, whose prefix and barrier would sit on its critical path,
// and workgroup 0 leaves the next call's hint from the exact active count instead (config
// [2] p = 0.001: 12.4 -> 11.6 us per step).  Integer sums make the result
// independent of R_eff and of the partition.  HBM traffic: the active rows' synapses once
// (E x (2 + 4 het) bytes) + R_eff partial rows of n_post x 4 bytes written and read (none
// at R_eff = 1).
#include <type_traits>

#include "common.h"

namespace {

constexpr int kBB = 256;          // build: threads per workgroup (one wave per row)
constexpr int kSB = 1024;         // step: threads per workgroup
constexpr int kMaxP = 12288;      // posts per bucket (48 KiB of 32-bit LDS accumulators)
constexpr int kMaxNb = 1024;      // buckets
// Measured on MI355X for 100k x 100k, K = 1000, p = 0.1: 9 buckets of 11,112
// posts with 28 row groups 30 us; 16 buckets 34 us; 32 buckets 48 us; 8 rows per wave with one
// pass 53 us; a 512-workgroup target 40 us.  fp32 LDS atomics instead of 64-bit integers:
// 76 us.
constexpr int kRowsPer = 4;       // active rows a wave works on at once
// the same in the fixed-grid dense kernel: measured for 100k x 100k, K = 1000 at p = 0.1 / 0.3 with 2, 4, 6, 8
// rows per wave: 28.4-28.6 / 55.5-56.2, 28.6-28.8 / 53.2-53.5, 29.2-29.4 / 54.3-54.5,
// 29.6-29.8 / 54.9-55.1 us per step
constexpr int kRowsDense = 4;
// the same in the single launch: measured for 100k x 100k, K = 1000 at p = 0.001 (~100 active rows) with
// 1 .. 8 rows per wave: 10.9, 10.2, 9.96, 10.9, 10.4, 10.6, 10.8, 11.0 us per step
constexpr int kRowsSingle = 3;
constexpr int kPasses = 2;        // 64-synapse passes per row issued together
constexpr int kSpan = 4096;       // active rows held in LDS before their synapses are added
constexpr int kTargetWgs = 256;   // step grid the row groups aim for
constexpr int kMinRows = 64;      // rows per row group, at least (and the group alignment)
constexpr int kMinNb = 8;         // buckets, at least (the grid is nb x row groups)
constexpr int kMaxR = kTargetWgs / kMinNb;  // row groups, at most (the reduce holds them all)
constexpr int kSample = 16384;    // leading spike rows whose active count sets R_eff
// active rows per row group the step aims for: measured for 100k x 100k, K = 1000 (mode 0, HIP graph)
// p = 0.003 / 0.01 with 256: 16.5 / 19.05 us, 128: 15.4 / 19.07 us (one box); on another,
// 256: 16.7 / 18.8 us, 64: 14.9 / 20.5 us
constexpr int kActivePer = 128;
constexpr int kDepth = 8;         // 16-byte spike loads per thread in flight together
constexpr int kHdr = 256;         // workspace bytes ahead of the partials (word 0: R_eff)
// single launch: workgroups per bucket.  Measured for 100k x 100k, K = 1000 at p = 0.001 (one launch of
// 9 x n workgroups): n = 2 13.0 us, 4 12.7 us, 8 12.55 us per step (HIP graph replay).
constexpr int kSubSingle = 8;

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

// Valid synapses onto each post (per-synapse weights: the D of the exponent rule below).
__global__ __launch_bounds__(kBB) void k_bucket_indeg(int32_t n_pre, const int32_t* indptr,
                                                      const int32_t* indices, int32_t k,
                                                      int32_t n_post, uint32_t* deg) {
  const int64_t s0 = indptr ? (int64_t)indptr[0] : 0;
  const int64_t s1 = indptr ? (int64_t)indptr[n_pre] : (int64_t)n_pre * k;
  for (int64_t s = s0 + (int64_t)blockIdx.x * kBB + threadIdx.x; s < s1;
       s += (int64_t)gridDim.x * kBB) {
    const int32_t t = indices[s];
    if ((uint32_t)t < (uint32_t)n_post) atomicAdd(&deg[t], 1u);
  }
}

__global__ void k_u32_fill0(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// The persistent runner's exponent rule, so that a projection stepped through this operator
// and the same projection inside the runner add the same integers: with W = max|w| over the
// valid synapses, W < 2^e_w (e_w from W's exponent field, -126 for a zero or subnormal W),
// and D = the largest number of valid synapses onto one post, D <= 2^e_d,
// S = min(30 - e_w - e_d, 100).  Every rounded weight is then an integer below 2^(30 - e_d)
// in magnitude, formed exactly in fp32 (ldexp, round to nearest even, convert), and every
// output's sum stays below 2^30 + D/2 (the runner sums in 32 bits, this operator in 64).
// -1000 flags a non-finite weight (or S < -100: weights too large for fixed point).
// One workgroup.
__global__ __launch_bounds__(kBB) void k_bucket_qexp(const uint32_t* wmax, const uint32_t* deg,
                                                     int32_t n_post, int32_t* qexp) {
  __shared__ uint32_t s_max[kBB / BS_WAVE];
  uint32_t m = 0u;
  for (int64_t j = threadIdx.x; j < n_post; j += kBB) m = deg[j] > m ? deg[j] : m;
  for (int o = BS_WAVE / 2; o > 0; o >>= 1) {
    const uint32_t v = (uint32_t)__shfl_xor((int)m, o);
    m = v > m ? v : m;
  }
  if (bs_lane() == 0) s_max[threadIdx.x / BS_WAVE] = m;
  __syncthreads();
  if (threadIdx.x != 0) return;
  uint32_t D = 0u;
  for (int w = 0; w < kBB / BS_WAVE; ++w) D = s_max[w] > D ? s_max[w] : D;
  const uint32_t bits = *wmax;
  const int e_w = (bits >> 23) ? (int)(bits >> 23) - 126 : -126;
  const int e_d = D <= 1u ? 0 : 32 - __clz(D - 1u);
  int S = 30 - e_w - e_d;
  if (S > 100) S = 100;
  *qexp = (bits >= 0x7F800000u || S < -100) ? -1000 : S;
}

// ---- step ----
// 16 bytes of spikes (16 u8 rows or 4 f32 rows) of block blk = rows [blk*E, blk*E + E), rows
// outside [r0, r1) read as 0: one vector load when the whole block lies inside and the
// vector is 16-byte aligned, else one load per row in range.
// The per-row form, out of line: it runs only for a block cut by the range or an unaligned
// vector, and kept inline its code (in every load slot) would be fetched by the instruction
// cache on every path (measured: 5x the misses of a compact kernel, ~2 us of a dense step).
template <typename T>
__device__ __noinline__ uint4 spike_block_rows(const T* __restrict__ spk, uint32_t row,
                                               uint32_t r0, uint32_t r1) {
  constexpr uint32_t kE = 16 / sizeof(T);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (uint32_t e = 0; e < kE; ++e) {
    const uint32_t i = row + e;
    if (i >= r0 && i < r1) {
      if (sizeof(T) == 1) w[e >> 2] |= (uint32_t)((const uint8_t*)spk)[i] << (8 * (e & 3));
      else w[e] = __float_as_uint(((const float*)spk)[i]);
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename T, bool kVec>
__device__ __forceinline__ uint4 spike_block(const T* __restrict__ spk, uint32_t blk, uint32_t r0,
                                             uint32_t r1) {
  constexpr uint32_t kE = 16 / sizeof(T);
  const uint32_t row = blk * kE;  // rows < 2^31: 32-bit index math (a 64-bit op costs two)
  if (kVec && row >= r0 && row + kE <= r1) return *(const uint4*)(spk + row);
  return spike_block_rows<T>(spk, row, r0, r1);
}

// Active rows of a block as a bit mask (u8: byte != 0; f32: value != 0, so -0 is inactive and
// NaN active, as `spk[i] != 0`), with word-parallel tests (a wave64 VALU op costs 4 cycles of
// its SIMD, and every lane tests 16 bytes per block):
//   u8:  bit 4k + q <-> byte k of word q = row 4q + k of the block (row_of below);
//   f32: bit q <-> row q.
template <typename T>
__device__ __forceinline__ uint32_t spike_bits(uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if (sizeof(T) == 1) {
    uint32_t u = 0u;  // byte k, bit q: byte k of word q is not zero
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // bit 8k+7 of y: byte k of the word is not zero (no carry leaves a byte)
      const uint32_t y = (((w[q] & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | w[q]) & 0x80808080u;
      u |= y >> (7 - q);
    }
    const uint32_t t = u | (u >> 4);            // byte 0: nibbles 0, 1; byte 2: nibbles 2, 3
    return (t & 0xFFu) | ((t >> 8) & 0xFF00u);
  }
  uint32_t m = 0u;
#pragma unroll
  for (int q = 0; q < 4; ++q) m |= (((w[q] & 0x7FFFFFFFu) + 0x7FFFFFFFu) >> 31) << q;
  return m;
}

// spike_bits, skipped (0) for the whole wave when none of its 64 blocks holds a non-zero
// word: two VALU ops and a ballot instead of the byte tests (sparse spikes leave many waves'
// blocks empty).
template <typename T>
__device__ __forceinline__ uint32_t spike_bits_sparse(uint4 v) {
  const bool any = (v.x | v.y | v.z | v.w) != 0u;
  return bs_ballot(any) != 0ull ? spike_bits<T>(v) : 0u;
}

// Row (inside its block) of bit e of spike_bits<T>.
template <typename T>
__device__ __forceinline__ int row_of(int e) {
  return sizeof(T) == 1 ? 4 * (e & 3) + (e >> 2) : e;
}

// Exclusive prefix over the wave's lanes of c (0 <= c < 2^kBits) and the wave's total, from
// the ballots of c's bits.
template <int kBits>
__device__ __forceinline__ void wave_prefix(uint32_t c, int& excl, int& total) {
  excl = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < kBits; ++k) {
    const uint64_t m = bs_ballot((c >> k) & 1u);
    excl += bs_rank_below(m) << k;
    total += (int)__popcll(m) << k;
  }
}

// Workgroup (b, r):
//   0. R_eff from the active count of the leading kSample rows (every workgroup reads the
//      same rows, so all agree); groups r >= R_eff return;
//   1. the group's rows in blocks of 16 bytes per thread, kDepth blocks' loads in flight;
//      each batch's active rows are appended to s_beg (ballot prefixes, one barrier);
//   2. when the list would pass kSpan rows, and at the end: every thread loads the bucket-b
//      bounds of some listed rows (all in flight) into s_beg / s_len;
//   3. waves take kRowsPer rows at a time and issue the loads of up to kPasses 64-synapse
//      passes of all of them before their LDS atomics;
//   4. R_eff = 1: the bucket's outputs, with k_bucket_reduce's arithmetic; else partial r.
template <typename T, bool kHet, bool kVec, bool kSingle>
__global__ __launch_bounds__(kSB) void k_bucket_scatter(
    const T* __restrict__ spk, int32_t n_pre, int32_t R, int32_t Rmax, int32_t nb, int32_t P,
    int32_t nsub,
    const int32_t* __restrict__ seg, const uint16_t* __restrict__ lidx,
    const float* __restrict__ lw, const int32_t* __restrict__ qexp, int32_t n_post,
    float w_homo, int32_t accumulate, float* __restrict__ out, int32_t* __restrict__ hdr,
    int32_t* __restrict__ est_out, uint32_t* __restrict__ part) {
  constexpr int kE = 16 / (int)sizeof(T);  // rows per block
  constexpr int kW = kSB / BS_WAVE;
  // fixed-point sums (two's complement; every sum is below 2^31 in magnitude by the choice of
  // S), fp32 sums or event counts
  __shared__ __align__(16) uint32_t s_acc32[kMaxP];
  __shared__ int32_t s_beg[kSpan];
  __shared__ int32_t s_len[kSpan];
  __shared__ int32_t s_wave[2][kW];
  const int lane = bs_lane();
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / BS_WAVE));
  // workgroup (b, sub, r): bucket b, sub-range sub of its posts (nsub > 1 only with R = 1),
  // row group r
  const int32_t b = blockIdx.x % nb;
  const int32_t sub = (blockIdx.x / nb) % nsub;
  const int32_t r = blockIdx.x / nb / nsub;
  // workgroup-wide exclusive prefix and total of c (< 2^kBits per thread), one barrier; s_wave
  // alternates halves, so the next call's writes never meet this call's reads
  int par = 0;
  auto prefix = [&](auto bits_tag, uint32_t c, int& excl, int& total) {
    int we, wt;
    wave_prefix<decltype(bits_tag)::value>(c, we, wt);
    if (lane == 0) s_wave[par][wid] = wt;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int v = 0; v < kW; ++v) {
      const int x = s_wave[par][v];
      base += v < wid ? x : 0;
      tot += x;
    }
    par ^= 1;
    excl = base + we;
    total = tot;
  };
  using B5 = std::integral_constant<int, 5>;   // counts of up to 16 rows
  using B8 = std::integral_constant<int, 8>;   // counts of up to 128 rows
  // fixed point (S >= -999) unless a weight is not finite; loaded first, so that its latency
  // hides behind the spike loads (a barrier waits for every outstanding scalar load)
  const int32_t S = kHet ? __builtin_amdgcn_readfirstlane(*qexp) : 0;
  // 0. R_eff = ceil(active rows / kActivePer), the active count estimated from the leading
  // ns rows (blocks d < kSmpD of every thread).  The first round of the group's rows is
  // loaded now too, before R_eff is known, on a guess that saves a memory round trip when it
  // holds: group 0 (which always starts at row 0) loads rows [0, n_pre) and clips them to its
  // end once R_eff is known; the other groups guess R_eff = R (the dense case) when their
  // group then fits the kDepth - kSmpD spare loads, and reload if the guess was wrong.
  constexpr int kSmpD = kSample / (kSB * kE);
  static_assert(kSmpD >= 1 && kSmpD < kDepth, "sample is part of the first round");
  const int32_t ns = n_pre < kSample ? n_pre : kSample;
  const uint32_t N = (uint32_t)n_pre;
  const uint32_t nblk = (N + kE - 1) / kE;
  // rows per group, a multiple of kMinRows (32-bit division: a 64-bit one is ~80 VALU ops,
  // and every wave of the workgroup computes it)
  auto group_rows = [&](int32_t groups) -> uint32_t {
    const uint32_t per = (N + (uint32_t)groups - 1u) / (uint32_t)groups;
    return (per + kMinRows - 1) / kMinRows * kMinRows;
  };
  // group r's rows when there are `groups` groups: [lo, hi) (64-bit product: r * rows may
  // pass 2^32 before the clamp)
  auto group_lo = [&](uint32_t rows) -> uint32_t {
    const uint64_t x = (uint64_t)r * rows;
    return x < N ? (uint32_t)x : N;
  };
  const uint32_t rowsR = group_rows(R);
  const uint32_t g0R = group_lo(rowsR);
  const uint32_t g1R = N - g0R > rowsR ? g0R + rowsR : N;
  const bool specR = r != 0 && rowsR <= (uint32_t)(kDepth - kSmpD) * kSB * kE;
  // v0[d]: d < kSmpD the sample, then group 0's or the R-guess's blocks (raw: their masks are
  // computed once R_eff says which of them the group needs)
  uint4 v0[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) {
    // slot d: uniform first block, row range and block limit; one compare per lane
    const uint32_t first = d < kSmpD || r == 0 ? (uint32_t)d * kSB
                                               : g0R / kE + (uint32_t)(d - kSmpD) * kSB;
    const uint32_t lo = d < kSmpD || r == 0 ? 0u : g0R;
    const uint32_t hi = d < kSmpD ? (uint32_t)ns : (r == 0 ? N : g1R);
    const uint32_t lim = d < kSmpD ? ((uint32_t)ns + kE - 1) / kE
                                   : (r == 0 ? nblk : (specR ? (g1R + kE - 1) / kE : 0u));
    const uint32_t blk = first + threadIdx.x;
    const bool want = blk < lim;
    v0[d] = want ? spike_block<T, kVec>(spk, blk, lo, hi) : make_uint4(0u, 0u, 0u, 0u);
  }
  // the bucket's LDS accumulator cleared while the loads are in flight (16-byte stores)
  // this workgroup's posts: [p0, p0 + pn), at offsets [lo_t, lo_t + pn) of bucket b
  const int32_t pnb = n_post - b * P < P ? n_post - b * P : P;  // posts in bucket b
  const int32_t ps = (P + nsub - 1) / nsub;
  const int32_t lo_t = sub * ps;
  const int32_t pn = pnb - lo_t < ps ? (pnb - lo_t > 0 ? pnb - lo_t : 0) : ps;
  const int32_t p0 = b * P + lo_t;
  for (int j = threadIdx.x; 4 * j < pn; j += kSB) ((uint4*)s_acc32)[j] = make_uint4(0u, 0u, 0u, 0u);
  uint32_t smk[kSmpD];  // masks of the sample's blocks
  uint32_t cs = 0;
#pragma unroll
  for (int d = 0; d < kSmpD; ++d) {
    smk[d] = spike_bits_sparse<T>(v0[d]);
    cs += __popc(smk[d]);
  }
  int32_t R_eff = 1;
  if constexpr (!kSingle) {  // the single launch (R = 1) needs no estimate to proceed
    int ex0, act0;
    prefix(B5(), cs, ex0, act0);
    // ceil(act0 * n_pre / (ns * kActivePer)) in double: the numerator (< 2^45) and the
    // denominator (<= 2^22) are exact, and a quotient that is not an integer lies at least
    // 2^-22 from one, far beyond the division's rounding, so the ceiling is exact
    const double re = ceil((double)act0 * (double)n_pre / ((double)ns * kActivePer));
    const int32_t est = re < 1.0 ? 1 : (re > (double)Rmax ? Rmax : (int32_t)re);
    R_eff = est < R ? est : R;  // R = 1: one launch, the step writes out
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      *hdr = R_eff;
      if (est_out) *est_out = est;  // the host's hint for its next call
    }
    if (r >= R_eff) return;  // whole workgroup
  } else {
    (void)cs;
  }
  const bool haveR = specR && R_eff == R;  // the R-guess held: mk0[kSmpD...] is the group
  const bool fixed = kHet && S > -1000;
  // the group's rows [g0, g1): R_eff groups, boundaries at multiples of kMinRows
  const uint32_t rows_g = group_rows(R_eff);
  const uint32_t g0 = group_lo(rows_g);
  const uint32_t g1 = N - g0 > rows_g ? g0 + rows_g : N;
  const uint32_t bk0 = g0 / kE, bk1 = (g1 + kE - 1) / kE;  // the group's blocks
  // masks of the first round read in phase 0, for the slots that hold blocks of the group
  // (a slot past the group's end is skipped whole: its mask work would be wasted)
  uint32_t mk0[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) {
    mk0[d] = 0u;
    if (r == 0) {
      const uint32_t blk = (uint32_t)d * kSB + threadIdx.x;
      if ((uint32_t)d * kSB < bk1 && blk < bk1)
        mk0[d] = d < kSmpD ? smk[d] : spike_bits_sparse<T>(v0[d]);
    } else if (haveR && d < kDepth - kSmpD) {
      const uint32_t blk = bk0 + (uint32_t)d * kSB + threadIdx.x;
      if ((uint32_t)d * kSB < bk1 - bk0 && blk < bk1) mk0[d] = spike_bits_sparse<T>(v0[kSmpD + d]);
    }
  }
  const int stride = nb + 1;
  int32_t count = 0;  // rows listed in s_beg (the same in every thread)
  uint32_t n_act = 0;  // active rows of the group (single launch: of all rows), every thread
  // bounds: s_beg holds rows (their bounds are loaded here); else s_beg / s_len hold the
  // rows' bounds already
  auto flush = [&](bool bounds = true) {
    __syncthreads();  // the listed rows are in s_beg
    // 2. bounds of bucket b in each listed row (count <= kSpan: all loads in flight)
    if (bounds) {
      constexpr int kU = kSpan / kSB;
      int32_t lo[kU], hi[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int32_t x = u * kSB + threadIdx.x;
        lo[u] = hi[u] = 0;
        if (x < count) {
          const int32_t* sr = seg + (uint64_t)(uint32_t)s_beg[x] * stride + b;
          lo[u] = sr[0];
          hi[u] = sr[1];
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int32_t x = u * kSB + threadIdx.x;
        if (x < count) {
          s_beg[x] = lo[u];
          s_len[x] = hi[u] - lo[u];
        }
      }
      __syncthreads();
    }
    // 3. synapses of kRP rows, up to kPasses x 64 each, loads in flight together
    constexpr int kRP = kSingle ? kRowsSingle : kRowsPer;
    for (int32_t a0 = wid * kRP; a0 < count; a0 += (kSB / BS_WAVE) * kRP) {
      int32_t beg[kRP], len[kRP];
      int32_t maxlen = 0;
#pragma unroll
      for (int q = 0; q < kRP; ++q) {
        const bool ok = a0 + q < count;
        beg[q] = ok ? s_beg[a0 + q] : 0;
        len[q] = ok ? s_len[a0 + q] : 0;
        maxlen = len[q] > maxlen ? len[q] : maxlen;
      }
      for (int32_t e0 = 0; e0 < maxlen; e0 += kPasses * BS_WAVE) {
        uint16_t t[kPasses][kRP];
        float v[kPasses][kRP];
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
#pragma unroll
          for (int q = 0; q < kRP; ++q) {
            const int32_t e = e0 + u * BS_WAVE + lane;
            t[u][q] = 0xFFFFu;
            v[u][q] = 0.0f;
            if (e < len[q]) {
              t[u][q] = lidx[(uint32_t)(beg[q] + e)];
              if (kHet) v[u][q] = lw[(uint32_t)(beg[q] + e)];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
#pragma unroll
          for (int q = 0; q < kRP; ++q) {
            // offset inside this workgroup's posts; the 0xFFFF of an idle lane is never < pn
            const uint32_t tl = (uint32_t)t[u][q] - (uint32_t)lo_t;
            if (tl < (uint32_t)pn) {
              if (!kHet) {
                atomicAdd(&s_acc32[tl], 1u);
              } else if (fixed) {
                const int32_t qv = (int32_t)__builtin_rintf(__builtin_ldexpf(v[u][q], S));
                atomicAdd(&s_acc32[tl], (uint32_t)qv);
              } else {
                atomicAdd((float*)&s_acc32[tl], v[u][q]);
              }
            }
          }
        }
      }
    }
    __syncthreads();  // s_beg / s_len are rewritten next
    count = 0;
  };
  // appends the rows of the set bits e of m at s_beg[pos...]: row0 + row_of(e), or, for
  // nibble q of a u8 mask (bit e <-> word e, byte q of the block), row0 + 4e + q
  auto put = [&](uint32_t m, uint32_t row0, int pos, int q) {
    while (m) {
      const int e = __builtin_ctz(m);
      s_beg[pos++] = (int32_t)(row0 + (q < 0 ? row_of<T>(e) : 4 * e + q));
      m &= m - 1u;
    }
  };
  // one batch (one block per thread) through the list, flushing it when it would overflow
  auto add_batch = [&](uint32_t m, uint32_t row0) {
    int ex, tot;
    prefix(B5(), (uint32_t)__popc(m), ex, tot);
    if (count + tot <= kSpan) {
      put(m, row0, count + ex, -1);
      count += tot;
      return;
    }
    if (count > 0) flush();
    if (tot <= kSpan) {
      put(m, row0, ex, -1);
      count = tot;
      return;
    }
    // more than kSpan active rows in one batch (u8 only): nibble by nibble, <= 4 per thread
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
      const uint32_t mq = (m >> (4 * q)) & 15u;
      int exq, totq;
      prefix(B5(), (uint32_t)__popc(mq), exq, totq);
      if (count + totq > kSpan) flush();
      put(mq, row0, count + exq, q);
      count += totq;
    }
  };
  // single launch, all rows in the first round: each thread loads the bucket bounds of up to
  // two of its active rows before the prefix that places them, so that round trip overlaps
  // the prefix's barrier and the list is complete after it (more rows in any thread, or more
  // than kSpan in all: the general path below).  For 100k x 100k, K = 1000 at p = 0.001 (a thread holds ~0.1
  // active rows; one with three or more turns up in ~14 % of spike vectors, which then take
  // ~12 us) 11.6 -> 11.0 us; up to three or four rows per thread (fallback in 0.4 % / 0.01 %)
  // measured 11.2 us.
  bool listed = false;
  if constexpr (kSingle) {
    if (r == 0 && bk1 - bk0 <= (uint32_t)kDepth * kSB) {
      uint32_t call = 0;
      int32_t rw[2] = {-1, -1};
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        uint32_t m = mk0[d];
        call += __popc(m);
        while (m) {
          const int e = __builtin_ctz(m);
          const int32_t row = (int32_t)(((uint32_t)d * kSB + threadIdx.x) * kE + row_of<T>(e));
          if (rw[0] < 0) rw[0] = row;
          else if (rw[1] < 0) rw[1] = row;
          m &= m - 1u;
        }
      }
      int32_t lo[2], hi[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        lo[q] = hi[q] = 0;
        if (rw[q] >= 0) {
          const int32_t* sr = seg + (uint64_t)(uint32_t)rw[q] * stride + b;
          lo[q] = sr[0];
          hi[q] = sr[1];
        }
      }
      // workgroup prefix of call, with "some thread has more than two rows" in bit 24 of
      // each wave's total (a wave lists at most 64 x 128 rows)
      int we, wt;
      wave_prefix<8>(call, we, wt);
      const bool many = bs_ballot(call > 2u) != 0ull;
      if (lane == 0) s_wave[par][wid] = wt | (many ? (1 << 24) : 0);
      __syncthreads();
      int base = 0, tot = 0, flag = 0;
#pragma unroll
      for (int v = 0; v < kW; ++v) {
        const int x = s_wave[par][v];
        base += v < wid ? (x & 0xFFFFFF) : 0;
        tot += x & 0xFFFFFF;
        flag |= x >> 24;
      }
      par ^= 1;
      if (!flag && tot <= kSpan) {
        const int ex = base + we;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (rw[q] >= 0) {
            s_beg[ex + q] = lo[q];
            s_len[ex + q] = hi[q] - lo[q];
          }
        }
        count = tot;
        n_act = (uint32_t)tot;
        listed = true;
      }
    }
  }
  // 1. the group's blocks, kDepth x kSB at a time: all loads first, then the whole round
  // through one prefix when its rows fit the list, else batch by batch
  for (uint32_t bb = listed ? bk1 : bk0; bb < bk1; bb += (uint32_t)kDepth * kSB) {
    uint32_t mk[kDepth];
    if (bb == bk0 && (r == 0 || haveR)) {  // read in phase 0
#pragma unroll
      for (int d = 0; d < kDepth; ++d) mk[d] = mk0[d];
    } else {
      uint4 v[kDepth];
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const uint32_t blk = bb + (uint32_t)d * kSB + threadIdx.x;
        v[d] = blk < bk1 ? spike_block<T, kVec>(spk, blk, g0, g1) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int d = 0; d < kDepth; ++d) mk[d] = spike_bits_sparse<T>(v[d]);
    }
    uint32_t call = 0;
#pragma unroll
    for (int d = 0; d < kDepth; ++d) call += __popc(mk[d]);
    int ex, tot;
    prefix(B8(), call, ex, tot);
    n_act += (uint32_t)tot;
    if (count + tot <= kSpan) {
      int pos = count + ex;
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        put(mk[d], (bb + (uint32_t)d * kSB + threadIdx.x) * kE, pos, -1);
        pos += __popc(mk[d]);
      }
      count += tot;
      continue;
    }
    const int nbat = (int)((bk1 - bb + kSB - 1) / kSB < kDepth ? (bk1 - bb + kSB - 1) / kSB
                                                                 : kDepth);
#pragma unroll 1
    for (int d = 0; d < nbat; ++d) {
      const uint32_t m = mk[0];
#pragma unroll
      for (int e = 0; e + 1 < kDepth; ++e) mk[e] = mk[e + 1];  // static indices: registers
      add_batch(m, (bb + (uint32_t)d * kSB + threadIdx.x) * kE);
    }
  }
  if (count > 0) flush(!listed);
  __syncthreads();  // s_acc complete (and zeroed, for a group without active rows)
  if (kSingle && blockIdx.x == 0 && threadIdx.x == 0) {  // the hint, from the exact count
    *hdr = 1;
    const uint32_t e = (n_act + kActivePer - 1) / kActivePer;
    if (est_out) *est_out = e < 1u ? 1 : (e > (uint32_t)Rmax ? Rmax : (int32_t)e);
  }
  // 4. output
  if (R_eff == 1) {
    float* o = out + p0;
    for (int j = threadIdx.x; j < pn; j += kSB) {
      float acc = accumulate ? o[j] : 0.0f;
      if (kHet && fixed) {
        const float v = ldexpf((float)(int32_t)s_acc32[j], -S);
        acc = accumulate ? acc + v : v;
      } else if (kHet) {
        acc += __uint_as_float(s_acc32[j]);
      } else {
        const uint32_t c = s_acc32[j];
        for (uint32_t u = 0; u < c; ++u) acc += w_homo;
      }
      o[j] = acc;
    }
  } else {
    uint32_t* dst = part + (int64_t)r * n_post + p0;
    for (int j = threadIdx.x; j < pn; j += kSB) dst[j] = s_acc32[j];
  }
}

// Dense spikes (mode 2: the previous call estimated the maximum R): every workgroup owns a
// fixed row group of `rows` rows, known on the host, so nothing waits for an estimate.  Per
// span of kSpan rows: kU spike bytes per thread and the bucket bounds of the active ones,
// loaded together, then ballots and one workgroup prefix that lists the active rows' bounds
// in ascending row order; then phase 3 as in the adaptive kernel.  This compact form is what
// dense steps are fastest with (100k x 100k, K = 1000 at p = 0.1: 31.6 us against 33.6 us for
// the adaptive kernel run at R = max).  Workgroup 0 writes R to the header and the next
// call's estimate from its own group's active rows.
template <typename T, bool kHet>
__global__ __launch_bounds__(kSB) void k_bucket_scatter_dense(
    const T* __restrict__ spk, int32_t n_pre, int32_t rows, int32_t R, int32_t Rmax, int32_t nb,
    int32_t P, const int32_t* __restrict__ seg, const uint16_t* __restrict__ lidx,
    const float* __restrict__ lw, const int32_t* __restrict__ qexp, int32_t n_post,
    int32_t* __restrict__ hdr, int32_t* __restrict__ est_out, uint32_t* __restrict__ part) {
  __shared__ uint32_t s_acc32[kMaxP];      // fixed-point sums, fp32 sums or event counts
  constexpr int kU = kSpan / kSB;          // span rows per thread
  __shared__ int32_t s_beg[kSpan];
  __shared__ int32_t s_len[kSpan];
  __shared__ int32_t s_wave[kU][kSB / BS_WAVE];
  const int lane = bs_lane();
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / BS_WAVE));
  const int32_t b = blockIdx.x % nb;
  const int32_t r = blockIdx.x / nb;
  const int32_t p0 = b * P;
  const int32_t pn = n_post - p0 < P ? n_post - p0 : P;  // posts in this bucket
  for (int j = threadIdx.x; j < pn; j += kSB) s_acc32[j] = 0u;
  // fixed point (S >= -999) unless a weight is not finite; scale = 2^S exactly
  const int32_t S = kHet ? __builtin_amdgcn_readfirstlane(*qexp) : 0;
  const bool fixed = kHet && S > -1000;
  const int64_t r0 = (int64_t)r * rows;
  const int64_t r1 = r0 + rows < n_pre ? r0 + rows : n_pre;
  const int stride = nb + 1;
  if (blockIdx.x == 0 && threadIdx.x == 0) *hdr = R;
  int32_t group_active = 0;  // active rows of the group (for workgroup 0's estimate)
  for (int64_t c0 = r0; c0 < r1; c0 += kSpan) {
    // 1+2. active rows of the span, ascending, with the bounds of bucket b in each: every
    // thread loads its kU spike bytes together and, for the active ones, the bounds, before
    // the one prefix that places them (one memory round trip and one barrier ahead of the
    // synapses, where a round per kSB rows took kU of each)
    int32_t lo[kU], hi[kU];
    uint64_t m[kU];
    {
      T sv[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t row = c0 + u * kSB + threadIdx.x;
        sv[u] = row < r1 ? spk[row] : T(0);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        lo[u] = hi[u] = 0;
        if (sv[u] != T(0)) {
          const int32_t* sr = seg + (c0 + u * kSB + threadIdx.x) * stride + b;
          lo[u] = sr[0];
          hi[u] = sr[1];
        }
        m[u] = bs_ballot(sv[u] != T(0));
        if (lane == 0) s_wave[u][wid] = __popcll(m[u]);
      }
    }
    __syncthreads();
    int32_t count = 0;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      int32_t pos = count, tot = 0;
#pragma unroll
      for (int v = 0; v < kSB / BS_WAVE; ++v) {
        pos += v < wid ? s_wave[u][v] : 0;
        tot += s_wave[u][v];
      }
      if ((m[u] >> lane) & 1ull) {
        pos += bs_rank_below(m[u]);
        s_beg[pos] = lo[u];
        s_len[pos] = hi[u] - lo[u];
      }
      count += tot;
    }
    group_active += count;
    __syncthreads();
    // 3. synapses of kRowsDense rows, up to kPasses x 64 each, loads in flight together
    for (int32_t a0 = wid * kRowsDense; a0 < count; a0 += (kSB / BS_WAVE) * kRowsDense) {
      int32_t beg[kRowsDense], len[kRowsDense];
      int32_t maxlen = 0;
#pragma unroll
      for (int q = 0; q < kRowsDense; ++q) {
        const bool ok = a0 + q < count;
        beg[q] = ok ? s_beg[a0 + q] : 0;
        len[q] = ok ? s_len[a0 + q] : 0;
        maxlen = len[q] > maxlen ? len[q] : maxlen;
      }
      for (int32_t e0 = 0; e0 < maxlen; e0 += kPasses * BS_WAVE) {
        uint16_t t[kPasses][kRowsDense];
        float v[kPasses][kRowsDense];
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
#pragma unroll
          for (int q = 0; q < kRowsDense; ++q) {
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
          for (int q = 0; q < kRowsDense; ++q) {
            if (t[u][q] != 0xFFFFu) {
              if (!kHet) {
                atomicAdd(&s_acc32[t[u][q]], 1u);
              } else if (fixed) {
                const int32_t qv = (int32_t)__builtin_rintf(__builtin_ldexpf(v[u][q], S));
                atomicAdd(&s_acc32[t[u][q]], (uint32_t)qv);
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
  if (blockIdx.x == 0 && threadIdx.x == 0 && est_out && r1 > r0) {
    // the next call's hint: the group's share of active rows, scaled to n_pre
    const double re = ceil((double)group_active * (double)n_pre /
                           ((double)(r1 - r0) * kActivePer));
    *est_out = re < 1.0 ? 1 : (re > (double)Rmax ? Rmax : (int32_t)re);
  }
  __syncthreads();
  uint32_t* dst = part + (int64_t)r * n_post + p0;
  for (int j = threadIdx.x; j < pn; j += kSB) dst[j] = s_acc32[j];
}

// out[j] = (accumulate ? out[j] : 0) + the bucket sums of j, over the R = *hdr partials the
// step kernel wrote (R = 1: it wrote out itself, nothing to do).  The first min(8, Rmax)
// partials are loaded together with the header, and the rest (R <= kMaxR) all together once R
// is known: two memory round trips in all (issued 8 at a time, then one by one, they took up
// to 7 at R = 28: 100k x 100k, K = 1000, p = 0.1 26.4 -> 25.4 us per call, p = 0.03 18.0 ->
// 17.0 us).
//   fixed point: the R partials added exactly (32-bit two's complement: every partial and the
//   total are below 2^31 in magnitude by the choice of S), then fl32(sum) * 2^-S;
//   homogeneous: the total count c of events, then c additions of w (the sequential chain);
//   fp32 fallback: the R partials added in row-group order.
template <bool kHet>
__global__ __launch_bounds__(256) void k_bucket_reduce(int32_t n_post, int32_t Rmax, int32_t Rfix,
                                                       const int32_t* __restrict__ hdr,
                                                       const uint32_t* __restrict__ part,
                                                       const int32_t* __restrict__ qexp,
                                                       float w_homo, int32_t accumulate,
                                                       float* __restrict__ out) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= n_post) return;
  constexpr int kFirst = 8;
  uint32_t x[kMaxR];   // the partials of j in row-group order (0 past R)
#pragma unroll
  for (int u = 0; u < kFirst; ++u) x[u] = u < Rmax ? part[(int64_t)u * n_post + j] : 0u;
  const int32_t S = kHet ? __builtin_amdgcn_readfirstlane(*qexp) : 0;
  float acc = accumulate ? out[j] : 0.0f;
  // Rfix > 0: the host fixed the row groups, no header to wait for
  const int32_t R = Rfix > 0 ? Rfix : __builtin_amdgcn_readfirstlane(*hdr);
  // (the loads above are consumed on both paths, so they stay ahead of this test)
  uint32_t any = __float_as_uint(acc) + (uint32_t)S;
#pragma unroll
  for (int u = 0; u < kFirst; ++u) any |= x[u];
  if (R <= 1 && any != 0x5A5A5A5Au) return;
  // the rest in one round trip: all loads issued before any is added
#pragma unroll
  for (int u = 0; u < kFirst; ++u)
    if (u >= R) x[u] = 0u;
#pragma unroll
  for (int u = kFirst; u < kMaxR; ++u) x[u] = u < R ? part[(int64_t)u * n_post + j] : 0u;
  if (kHet && S > -1000) {
    uint32_t q = 0;   // wrap-around adds: the true sum fits, so the result is exact
#pragma unroll
    for (int u = 0; u < kMaxR; ++u) q += x[u];
    const float v = ldexpf((float)(int32_t)q, -S);
    acc = accumulate ? acc + v : v;
  } else if (kHet) {
    // fp32 fallback: the partials in row-group order
#pragma unroll
    for (int u = 0; u < kMaxR; ++u)
      if (u < R) acc += __uint_as_float(x[u]);
  } else {
    uint32_t c = 0;
#pragma unroll
    for (int u = 0; u < kMaxR; ++u) c += x[u];
    for (uint32_t u = 0; u < c; ++u) acc += w_homo;
  }
  out[j] = acc;
}

int32_t row_groups(int32_t n_pre, int32_t nb) {
  int64_t R = kTargetWgs / (nb > 0 ? nb : 1);
  if (R > kMaxR) R = kMaxR;  // fewer than kMinNb buckets (a caller's own layout, tiny n_post)
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
               "bs_bucket_build: per-synapse weights need qexp and a workspace of "
               "4 * (n_post + 1) bytes");
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
    if (w) {  // no synapse: W = 0, D = 0
      k_u32_fill0<<<1, 256, 0, s>>>((uint32_t*)workspace, 1);
      BS_CHECK_LAUNCH();
      k_bucket_qexp<<<1, kBB, 0, s>>>((uint32_t*)workspace, nullptr, 0, qexp);
      BS_CHECK_LAUNCH();
    }
    return BS_OK;
  }
  uint32_t* wmax = (uint32_t*)workspace;
  uint32_t* deg = wmax + 1;  // [n_post] valid synapses onto each post
  if (w) {
    k_u32_fill0<<<256, 256, 0, s>>>(wmax, (int64_t)n_post + 1);
    BS_CHECK_LAUNCH();
    k_bucket_indeg<<<2048, kBB, 0, s>>>(n_pre, indptr, indices, k, n_post, deg);
    BS_CHECK_LAUNCH();
  }
  k_bucket_place<<<(int)g, kBB, shm, s>>>(n_pre, indptr, indices, w, k, n_post, nb, P, seg, lidx,
                                          lw, w ? wmax : nullptr);
  BS_CHECK_LAUNCH();
  if (w) {
    k_bucket_qexp<<<1, kBB, 0, s>>>(wmax, deg, n_post, qexp);
    BS_CHECK_LAUNCH();
  }
  return BS_OK;
}

extern "C" size_t bs_event_bucket_workspace_size(int32_t n_pre, int32_t n_post, int32_t nb) {
  bs_clear_error();
  if (n_pre <= 0 || n_post <= 0 || nb <= 0) return 0;
  return (size_t)kHdr + (size_t)row_groups(n_pre, nb) * n_post * sizeof(uint32_t);
}

extern "C" int bs_event_bucket_f32(const void* spk, int32_t spk_dtype, int32_t n_pre,
                                   int32_t n_post, int32_t nb, int32_t P, const int32_t* seg,
                                   const uint16_t* lidx, const float* lw, const int32_t* qexp,
                                   float w_homo, float* out, int32_t accumulate, void* workspace,
                                   size_t workspace_bytes, int32_t mode, int32_t* est_out,
                                   bs_stream_t stream) {
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
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || (uintptr_t)spk % sizeof(float) == 0,
               "bs_event_bucket_f32: f32 spikes not 4-byte aligned");
  BS_CHECK_ARG(lw == nullptr || qexp != nullptr, "bs_event_bucket_f32: qexp is NULL");
  BS_CHECK_ARG(mode >= 0 && mode <= 2, "bs_event_bucket_f32: mode %d outside [0, 2]", mode);
  const int32_t Rmax = row_groups(n_pre, nb);
  const bool single_launch = mode == 1;
  // the fixed-grid kernel only writes partials: with a single row group (Rmax = 1) there is
  // nothing for the reduce to add, so that case runs as mode 0, whose one group writes out
  const bool dense = mode == 2 && Rmax > 1;
  const int32_t R = single_launch ? 1 : Rmax;  // one group per bucket: no partials, no reduce
  // single launch: each bucket's posts split over nsub workgroups (every one scans the spikes
  // and the bucket's synapses, and adds and writes only its slice)
  // every workgroup of the single launch scans the whole spike vector: at most kSubSingle
  // per bucket, and about kTargetWgs in all when there are many buckets
  int32_t nsub = 1;
  if (single_launch) {
    nsub = kTargetWgs / nb < kSubSingle ? kTargetWgs / nb : kSubSingle;
    if (nsub > P) nsub = P;
    if (nsub < 1) nsub = 1;
  }
  const size_t need = (size_t)kHdr + (single_launch ? 0 : (size_t)R * n_post * sizeof(uint32_t));
  BS_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "bs_event_bucket_f32: workspace of %zu bytes needed (got %zu)", need,
               workspace ? workspace_bytes : (size_t)0);
  BS_CHECK_ARG((uintptr_t)workspace % 8 == 0,
               "bs_event_bucket_f32: workspace not 8-byte aligned");
  int32_t* hdr = (int32_t*)workspace;  // R_eff, written by the step kernel
  uint32_t* part = (uint32_t*)((char*)workspace + kHdr);
  const int64_t g = (int64_t)nb * nsub * R;
  const bool vec = (uintptr_t)spk % 16 == 0;  // 16-byte spike loads
#define BS_BK(T, H, V)                                                                      \
  do {                                                                                      \
    if (single_launch)                                                                      \
      k_bucket_scatter<T, H, V, true><<<(int)g, kSB, 0, s>>>(                               \
          (const T*)spk, n_pre, R, Rmax, nb, P, nsub, seg, lidx, lw, qexp, n_post, w_homo,   \
          accumulate, out, hdr, est_out, part);                                             \
    else                                                                                    \
      k_bucket_scatter<T, H, V, false><<<(int)g, kSB, 0, s>>>(                              \
          (const T*)spk, n_pre, R, Rmax, nb, P, nsub, seg, lidx, lw, qexp, n_post, w_homo,   \
          accumulate, out, hdr, est_out, part);                                             \
  } while (0)
#define BS_BK2(T, H) \
  do { if (vec) BS_BK(T, H, true); else BS_BK(T, H, false); } while (0)
#define BS_BD(T, H)                                                                         \
  k_bucket_scatter_dense<T, H><<<(int)g, kSB, 0, s>>>((const T*)spk, n_pre, rows, R, Rmax, nb, P, \
                                                      seg, lidx, lw, qexp, n_post, hdr, est_out, \
                                                      part)
  if (dense) {
    const int32_t rows = (int32_t)(((int64_t)n_pre + R - 1) / R);
    if (spk_dtype == BS_SPK_U8) { if (lw) BS_BD(uint8_t, true); else BS_BD(uint8_t, false); }
    else { if (lw) BS_BD(float, true); else BS_BD(float, false); }
  } else if (spk_dtype == BS_SPK_U8) {
    if (lw) BS_BK2(uint8_t, true); else BS_BK2(uint8_t, false);
  } else {
    if (lw) BS_BK2(float, true); else BS_BK2(float, false);
  }
#undef BS_BD
#undef BS_BK2
#undef BS_BK
  BS_CHECK_LAUNCH();
  if (single_launch) return BS_OK;
  const int gr = (int)(((int64_t)n_post + 255) / 256);
  if (lw)
    k_bucket_reduce<true><<<gr, 256, 0, s>>>(n_post, R, dense ? R : 0, hdr, part, qexp, w_homo,
                                             accumulate, out);
  else
    k_bucket_reduce<false><<<gr, 256, 0, s>>>(n_post, R, dense ? R : 0, hdr, part, qexp, w_homo,
                                              accumulate, out);
  BS_CHECK_LAUNCH();
  return BS_OK;
}

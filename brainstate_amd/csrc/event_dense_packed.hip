// Batched event x dense weight on the matrix cores, exact in fixed point: EventLinear with a
// weight matrix that is packed once and reused across calls (a recurrent run, inference).
//
// out[b, j] = sum of W[i, j] over the inputs i with spk[b, i] != 0.
//
// Arithmetic.  Column j of W is scaled by 2^S_j, fixed by its largest magnitude
// m_j = max_i |W[i, j]| = f * 2^e_j (f in [0.5, 1)): S_j = D - e_j with D = 8 L - 2, so each
// q[i, j] = rint(W[i, j] * 2^S_j) (ties to even) has |q| <= 2^D.  L, the number of signed
// 8-bit digits that hold q, is the smallest with D >= 24 + ceil(log2 n_in); the rounding of
// the weights then moves a sum by at most n_in * 2^(e_j - D - 1) <= 2^-24 * m_j.  The sums of
// q over the active inputs are exact integers (so their order does not matter) and are
// rounded once: out = ldexp((float) sum, -S_j).  A column of zeros gives +0.
//
// Digits: q = sum_l d_l * 256^l with every d_l in [-128, 127] (d_0 = q mod 256 read as a
// signed byte, then the same for (q - d_0) / 256, ...).  The 0/1 spike bytes times the
// digits run on v_mfma_i32_16x16x64_i8 (16 batch rows x 16 columns x 64 inputs per
// instruction) with one int32 accumulator per digit (|acc| <= 128 n_in), and the digit sums
// are combined in int64 (|sum| <= n_in * 2^D <= 2^62 for n_in <= 65536).
//
// Packed layout (bs_event_dense_pack): a 256-byte header whose first int32 is the status
// (0, or 1 when a weight is not finite), then the bit patterns of m_j for the NT * 16 padded
// columns (uint32; NT = ceil(n_out / 16); rounded up to 256 bytes), then the digits in
// 1024-byte blocks, one per (column tile t, input block k of 64 inputs, digit l), at
// ((t * KB + k) * L + l) * 1024, KB = ceil(n_in / 64) rounded up to a multiple of 8.  Byte 16 m + u of a block is digit l of
// W[64 k + 16 (m / 16) + u, 16 t + m % 16]: lane m of the instruction's B operand holds
// column m % 16, and the spike operand puts batch row m % 16 and the same 16 inputs in lane
// m, so both operands agree on which input each byte is (the instruction sums over all 64
// inputs of the block, so only that agreement matters).  Padding rows and columns hold zero
// digits.
//
// Forward tiling: a workgroup owns one column tile of 16 columns and 64 batch rows (4 MFMA
// row tiles; tiles ordered so that neighbours share an XCD); its 4 waves split the input
// blocks into 4 consecutive ranges and stream their
// digit blocks (16 bytes per lane per digit, 1 KiB per wave-load) with the next group of
// blocks in flight while the current one is multiplied.  The waves' int64 sums meet in LDS
// and wave w rounds and stores row tile w.
#include "bs_math.h"
#include "common.h"
#include "neuron_dev.h"

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));

constexpr int kHeader = 256;
constexpr int kBlkIn = 64;      // inputs per instruction (K)
constexpr int kTileN = 16;      // columns per tile (N)
constexpr int kRowTiles = 4;    // row tiles of 16 per workgroup
constexpr int kGroupB = 16 * kRowTiles;   // batch rows per workgroup
constexpr int kPW = kRowTiles;  // waves per workgroup (waves 0..3 store row tiles 0..3)
constexpr int kPB = kPW * BS_WAVE;
constexpr int kGroup = 2;       // input blocks per pipeline stage
constexpr int32_t kMaxIn = 65536;
constexpr int kMaxRowsWg = 256; // column-maximum pass: rows per workgroup

int ceil_log2(int64_t n) {
  int c = 0;
  while ((1LL << c) < n) ++c;
  return c;
}

// Smallest L in 4..6 with 8 L - 2 >= 24 + ceil(log2 n_in); 0 when n_in is out of range.
int digits_for(int32_t n_in) {
  if (n_in < 0 || n_in > kMaxIn) return 0;
  const int c = ceil_log2(n_in > 0 ? n_in : 1);
  for (int L = 4; L <= 6; ++L)
    if (8 * L - 2 >= 24 + c) return L;
  return 0;
}

struct PackDims {
  int32_t L, KB, NT;
  int64_t bits_off, dig_off, total;
};

PackDims pack_dims(int32_t n_in, int32_t n_out) {
  PackDims d;
  d.L = digits_for(n_in);
  // input blocks, padded with zero digits to whole pipeline stages of every wave
  constexpr int kStageBlocks = kPW * kGroup;
  d.KB = ((n_in + kBlkIn - 1) / kBlkIn + kStageBlocks - 1) / kStageBlocks * kStageBlocks;
  d.NT = (n_out + kTileN - 1) / kTileN;
  d.bits_off = kHeader;
  d.dig_off = kHeader + ((int64_t)d.NT * kTileN * 4 + 255) / 256 * 256;
  d.total = d.dig_off + (int64_t)d.NT * d.KB * d.L * 1024;
  return d;
}

// frexp exponent of a positive finite float given by its bits (bits != 0).
__device__ __forceinline__ int frexp_exp_bits(uint32_t mb) {
  const int E = (int)(mb >> 23);
  if (E != 0) return E - 126;
  return (31 - __builtin_clz(mb)) - 148;  // subnormal: mant in [2^p, 2^(p+1)) -> p - 148
}

// rint(x * 2^S) for a finite float x, exactly, from its bits (no dependence on the
// floating-point denormal mode): x = +-M * 2^(E' - 150), so x * 2^S = +-M * 2^sh.
__device__ __forceinline__ int64_t fixed_bits(uint32_t xb, int S) {
  const uint32_t E = (xb >> 23) & 255u;
  const uint32_t mant = xb & 0x7fffffu;
  const int64_t M = E ? (int64_t)(mant | 0x800000u) : (int64_t)mant;
  const int sh = (E ? (int)E : 1) - 150 + S;
  int64_t q;
  if (sh >= 0) {
    q = M << sh;  // |q| <= 2^D: sh <= D - 23 here
  } else if (sh < -25) {
    q = 0;        // |x * 2^S| < 2^-1
  } else {
    const int r = -sh;
    const int64_t t = M >> r, rem = M & ((1LL << r) - 1), half = 1LL << (r - 1);
    q = t + ((rem > half || (rem == half && (t & 1))) ? 1 : 0);  // ties to even
  }
  return (xb >> 31) ? -q : q;
}

__global__ void k_pack_clear(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Column maxima of |W| as bit patterns (non-negative floats order like their bits); a
// non-finite weight sets the status word.  Workgroup: 64 columns x kMaxRowsWg rows.
__global__ __launch_bounds__(256) void k_pack_colmax(const float* __restrict__ W, int32_t n_in,
                                                     int32_t n_out, uint32_t* status,
                                                     uint32_t* bits) {
  __shared__ uint32_t s_m[4][64];
  const int cl = threadIdx.x & 63, s = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + cl;
  const int64_t r0 = (int64_t)blockIdx.y * kMaxRowsWg;
  const int64_t r1 = r0 + kMaxRowsWg < n_in ? r0 + kMaxRowsWg : n_in;
  uint32_t m = 0;
  bool bad = false;
  if (c < n_out) {
    for (int64_t r = r0 + s; r < r1; r += 4) {
      const uint32_t u = __float_as_uint(W[r * n_out + c]) & 0x7fffffffu;
      bad |= u >= 0x7f800000u;
      m = m > u ? m : u;
    }
  }
  if (bad) atomicOr(status, 1u);
  s_m[s][cl] = m;
  __syncthreads();
  if (s == 0 && c < n_out) {
    uint32_t a = s_m[0][cl] > s_m[1][cl] ? s_m[0][cl] : s_m[1][cl];
    const uint32_t b = s_m[2][cl] > s_m[3][cl] ? s_m[2][cl] : s_m[3][cl];
    a = a > b ? a : b;
    if (a != 0u) atomicMax(bits + c, a);
  }
}

// Digits: thread = (padded column c, group g of 16 inputs); consecutive threads take
// consecutive columns, so the W reads of a wave are coalesced and its 16-byte digit stores
// fill whole 256-byte runs of a block.
template <int L>
__global__ __launch_bounds__(256) void k_pack_digits(const float* __restrict__ W, int32_t n_in,
                                                     int32_t n_out, int32_t KB, int32_t NT,
                                                     const uint32_t* __restrict__ bits,
                                                     uint8_t* __restrict__ dig) {
  constexpr int D = 8 * L - 2;
  const int64_t ncol = (int64_t)NT * kTileN;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t c = tid % ncol, g = tid / ncol;
  if (g >= (int64_t)KB * 4) return;
  const uint32_t mb = c < n_out ? bits[c] : 0u;
  const int S = mb ? D - frexp_exp_bits(mb) : 0;
  uint32_t w[L][4];
#pragma unroll
  for (int l = 0; l < L; ++l) w[l][0] = w[l][1] = w[l][2] = w[l][3] = 0u;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int64_t r = g * 16 + u;
    uint32_t xb = 0u;
    if (c < n_out && r < n_in) xb = __float_as_uint(W[r * n_out + c]);
    int64_t q = (mb && (xb & 0x7fffffffu) < 0x7f800000u) ? fixed_bits(xb, S) : 0;
#pragma unroll
    for (int l = 0; l < L; ++l) {
      const int64_t d = (int64_t)(int8_t)(uint8_t)(q & 255);
      q = (q - d) >> 8;  // exact: q - d is a multiple of 256
      w[l][u >> 2] |= ((uint32_t)d & 255u) << (8 * (u & 3));
    }
  }
  const int64_t t = c >> 4, k = g >> 2;
  const int m = 16 * (int)(g & 3) + (int)(c & 15);
#pragma unroll
  for (int l = 0; l < L; ++l)
    *(uint4*)(dig + ((t * KB + k) * L + l) * 1024 + m * 16) =
        make_uint4(w[l][0], w[l][1], w[l][2], w[l][3]);
}

// 0x01 in each byte of x that is nonzero, 0x00 elsewhere.
__device__ __forceinline__ uint32_t nz_bytes(uint32_t x) {
  return ((((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x) >> 7) & 0x01010101u;
}

// Spike operand of one row tile for input block k: lane holds batch row b, inputs
// 64 k + 16 (lane / 16) + [0, 16) as 0/1 bytes.
template <typename T, bool kVec>
__device__ __forceinline__ v4i load_spk(const T* __restrict__ spk, int32_t batch, int32_t n_in,
                                        int32_t b, int64_t i0) {
  v4i a = {0, 0, 0, 0};
  if (b >= batch || i0 >= n_in) return a;
  const T* p = spk + (int64_t)b * n_in + i0;
  if constexpr (sizeof(T) == 1) {
    if (kVec) {  // n_in % 16 == 0 and 16-byte aligned rows: i0 + 16 <= n_in
      const uint4 x = *(const uint4*)p;
      a[0] = (int32_t)nz_bytes(x.x);
      a[1] = (int32_t)nz_bytes(x.y);
      a[2] = (int32_t)nz_bytes(x.z);
      a[3] = (int32_t)nz_bytes(x.w);
    } else {
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (i0 + u < n_in && p[u] != 0) a[u >> 2] |= 1 << (8 * (u & 3));
    }
  } else {
    if (kVec) {  // n_in % 16 == 0 and 16-byte aligned rows
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 x = *(const float4*)(p + 4 * q);
        a[q] = (x.x != 0.0f ? 1 : 0) | (x.y != 0.0f ? 1 << 8 : 0) |
               (x.z != 0.0f ? 1 << 16 : 0) | (x.w != 0.0f ? 1 << 24 : 0);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (i0 + u < n_in && p[u] != 0.0f) a[u >> 2] |= 1 << (8 * (u & 3));
    }
  }
  return a;
}

// COBA-LIF state of the fused step (bs_event_dense_packed_lif_step); unused otherwise.
struct LifOut {
  float* V;
  float* ge;
  float* gi;
  int32_t* ref;
  uint8_t* spk;
  int32_t inh;  // the product drives g_i (1) or g_e (0)
  bs_lif_params p;
};

template <typename T, int L, bool kVec, bool kLif>
__global__ __launch_bounds__(kPB) void k_event_dense_packed(
    const T* __restrict__ spk, int32_t batch, int32_t n_in, const uint8_t* __restrict__ dig,
    const uint32_t* __restrict__ bits, const uint32_t* __restrict__ status, int32_t n_out,
    int32_t KB, float* __restrict__ out, LifOut lif) {
  constexpr int D = 8 * L - 2;
  __shared__ int64_t s_sum[kPW][kRowTiles][4][BS_WAVE];  // 8 KiB per wave
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin; consecutive tiles
  // share an XCD (and its L2), so the two 64-byte halves of each 128-byte line of the
  // outputs and neuron state meet in one L2 (fused step 19.2 -> 18.5 us for 64 x 4096
  // spikes and a 4096 x 4096 W)
  const int64_t nt = gridDim.x, per = (nt + 7) / 8;
  const int64_t bx = blockIdx.x, xcd = bx % 8, slot = bx / 8;
  const int64_t full = nt % 8 == 0 ? 8 : nt % 8;  // XCDs that hold `per` tiles
  const int64_t t = xcd < full ? xcd * per + slot : full * per + (xcd - full) * (per - 1) + slot;
  const int32_t b0 = (int32_t)blockIdx.y * kGroupB;
  const int32_t k_lo = (int32_t)((int64_t)KB * wid / kPW);
  const int32_t k_hi = (int32_t)((int64_t)KB * (wid + 1) / kPW);
  const uint8_t* dp = dig + t * KB * L * 1024 + lane * 16;
  const int32_t brow = b0 + (lane & 15);
  const int64_t iq = (lane >> 4) * 16;

  v4i acc[kRowTiles][L];
#pragma unroll
  for (int mt = 0; mt < kRowTiles; ++mt)
#pragma unroll
    for (int l = 0; l < L; ++l) acc[mt][l] = v4i{0, 0, 0, 0};

  // fused step: the neuron state of the outputs this lane will finish is loaded now, so its
  // latency passes while the digits stream (loaded after the last digit loads instead, it is
  // left exposed: the last products are too short to cover it, 17.9 -> 18.7 us)
  const int64_t j = t * kTileN + (lane & 15);
  float sV[4], sge[4], sgi[4];
  int32_t sref[4];
  if constexpr (kLif) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t b = b0 + 16 * wid + 4 * (lane >> 4) + r;
      const bool v = wid < kRowTiles && b < batch && j < n_out;
      const int64_t o = v ? (int64_t)b * n_out + j : 0;
      sV[r] = v ? lif.V[o] : 0.0f;
      sge[r] = v ? lif.ge[o] : 0.0f;
      sgi[r] = v ? lif.gi[o] : 0.0f;
      sref[r] = v ? lif.ref[o] : 0;
    }
  }

  // one pipeline stage: kGroup input blocks.  Every wave's block range is whole stages (KB is
  // a multiple of kPW * kGroup), so no stage reaches past it.  Byte spikes on the 16-byte path
  // are loaded from clamped addresses (rows past `batch` repeat the last row, whose sums are
  // never stored; inputs past n_in repeat the last 16, whose digits are zero), kept raw and
  // masked when multiplied, so the loads need no masks or branches and none waits for another.
  constexpr bool kRaw = sizeof(T) == 1 && kVec;
  auto load = [&](int32_t k, v4i (&a)[kGroup][kRowTiles], v4i (&bv)[kGroup][L]) {
#pragma unroll
    for (int s = 0; s < kGroup; ++s) {
      const int64_t kk = k + s;
#pragma unroll
      for (int l = 0; l < L; ++l) bv[s][l] = *(const v4i*)(dp + (kk * L + l) * 1024);
      const int64_t i0 = kk * kBlkIn + iq;
#pragma unroll
      for (int mt = 0; mt < kRowTiles; ++mt) {
        const int32_t b = brow + 16 * mt;
        if constexpr (kRaw) {
          const int64_t off = (int64_t)(b < batch ? b : batch - 1) * n_in +
                              (i0 < n_in ? i0 : (int64_t)n_in - 16);
          a[s][mt] = *(const v4i*)((const uint8_t*)spk + off);
        } else {
          a[s][mt] = load_spk<T, kVec>(spk, batch, n_in, b, i0);
        }
      }
    }
  };
  auto mult = [&](const v4i (&a)[kGroup][kRowTiles], const v4i (&bv)[kGroup][L]) {
#pragma unroll
    for (int s = 0; s < kGroup; ++s)
#pragma unroll
      for (int mt = 0; mt < kRowTiles; ++mt) {
        v4i x = a[s][mt];
        if constexpr (kRaw) {
#pragma unroll
          for (int q = 0; q < 4; ++q) x[q] = (int32_t)nz_bytes((uint32_t)x[q]);
        }
#pragma unroll
        for (int l = 0; l < L; ++l)
          acc[mt][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, bv[s][l], acc[mt][l], 0, 0, 0);
      }
  };
  if (k_lo < k_hi) {
    // the steady-state body always has the next stage's loads in flight while it multiplies,
    // and every path into its first multiply has issued the same loads, so the waits before
    // each product count only the stage it needs; the last one or two stages follow it.  The
    // scheduling barriers keep each stage's loads together, ahead of the products they overlap
    // (left to itself the scheduler sinks them between the products, next to their first use,
    // and the waits shrink to the last few loads: product 17.0 -> 16.2 us for the same shape)
    auto sched = [] { __builtin_amdgcn_sched_barrier(0); };
    v4i a0[kGroup][kRowTiles], b0v[kGroup][L], a1[kGroup][kRowTiles], b1v[kGroup][L];
    load(k_lo, a0, b0v);
    int32_t k = k_lo;
    for (; k + 2 * kGroup < k_hi; k += 2 * kGroup) {
      sched(); load(k + kGroup, a1, b1v); sched();
      mult(a0, b0v);
      sched(); load(k + 2 * kGroup, a0, b0v); sched();
      mult(a1, b1v);
    }
    if (k + kGroup < k_hi) {
      sched(); load(k + kGroup, a1, b1v); sched();
      mult(a0, b0v);
      mult(a1, b1v);
    } else {
      mult(a0, b0v);
    }
  }

  // digit sums -> int64 (lane holds column lane % 16, rows 4 (lane / 16) + r of each tile)
#pragma unroll
  for (int mt = 0; mt < kRowTiles; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int64_t sum = 0;
#pragma unroll
      for (int l = 0; l < L; ++l) sum += (int64_t)acc[mt][l][r] * (int64_t)(1LL << (8 * l));
      s_sum[wid][mt][r][lane] = sum;
    }
  __syncthreads();
  const int mt = wid;
  if (mt >= kRowTiles || j >= n_out) return;
  const uint32_t mb = bits[j];
  const bool bad = *status != 0u;
  const int S = mb ? D - frexp_exp_bits(mb) : 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int32_t b = b0 + 16 * mt + 4 * (lane >> 4) + r;
    if (b >= batch) continue;
    int64_t tot = 0;
#pragma unroll
    for (int w = 0; w < kPW; ++w) tot += s_sum[w][mt][r][lane];
    float v = mb ? ldexpf((float)tot, -S) : 0.0f;
    if (bad) v = __builtin_nanf("");
    const int64_t o = (int64_t)b * n_out + j;
    if (!kLif || out != nullptr) out[o] = v;
    if constexpr (kLif) {
      // the update of bs_coba_lif_step with this output as its conductance input
      float V = sV[r], ge = sge[r], gi = sgi[r];
      int32_t rf = sref[r];
      const float in_e = lif.inh ? 0.0f : v, in_i = lif.inh ? v : 0.0f;
      const bool sp = bs_lif_update_p(lif.p, V, ge, gi, rf, in_e, in_i);
      lif.V[o] = V;
      lif.ge[o] = ge;
      lif.gi[o] = gi;
      lif.ref[o] = rf;
      if (lif.spk != nullptr) lif.spk[o] = sp ? 1 : 0;
    }
  }
}

template <typename T, int L>
void launch_packed(const T* spk, int32_t batch, int32_t n_in, const PackDims& d,
                   const uint8_t* packed, int32_t n_out, float* out, bool vec,
                   const LifOut* lif, hipStream_t s) {
  const dim3 grid(d.NT, (batch + kGroupB - 1) / kGroupB);
  const uint8_t* dig = packed + d.dig_off;
  const uint32_t* bits = (const uint32_t*)(packed + d.bits_off);
  const uint32_t* status = (const uint32_t*)packed;
  const LifOut none{};
#define BS_PK(V, F)                                                                        \
  k_event_dense_packed<T, L, V, F><<<grid, kPB, 0, s>>>(spk, batch, n_in, dig, bits, status, \
                                                        n_out, d.KB, out, F ? *lif : none)
  if (lif) { if (vec) BS_PK(true, true); else BS_PK(false, true); }
  else { if (vec) BS_PK(true, false); else BS_PK(false, false); }
#undef BS_PK
}

// Checks shared by the two product entry points; dispatch on the spike type and L.
int packed_product(const char* fn, const void* spk, int32_t spk_dtype, int32_t batch,
                   int32_t n_in, const void* packed, int32_t n_out, float* out,
                   const LifOut* lif, hipStream_t s) {
  BS_CHECK_ARG(batch >= 0 && n_in >= 0 && n_out >= 0, "%s: negative size", fn);
  BS_CHECK_ARG(n_in <= kMaxIn, "%s: n_in = %d exceeds %d", fn, n_in, kMaxIn);
  BS_CHECK_ARG(spk_dtype == BS_SPK_U8 || spk_dtype == BS_SPK_F32,
               "%s: unknown spike dtype %d", fn, spk_dtype);
  BS_CHECK_ARG(packed != nullptr && ((uintptr_t)packed & 255) == 0,
               "%s: packed buffer must be non-NULL and 256-byte aligned", fn);
  BS_CHECK_ARG((batch + kGroupB - 1) / kGroupB <= 65535, "%s: batch %d too large", fn, batch);
  if ((int64_t)batch * n_out == 0) return BS_OK;
  BS_CHECK_ARG(out != nullptr || lif != nullptr, "%s: out is NULL", fn);
  BS_CHECK_ARG(spk != nullptr || n_in == 0, "%s: spk is NULL", fn);
  const PackDims d = pack_dims(n_in, n_out);
  const uint8_t* pk = (const uint8_t*)packed;
  const size_t es = spk_dtype == BS_SPK_U8 ? 1 : 4;
  const bool vec = n_in % 16 == 0 && ((uintptr_t)spk & 15) == 0 && (n_in * es) % 16 == 0;
  if (spk_dtype == BS_SPK_U8) {
    const uint8_t* p = (const uint8_t*)spk;
    switch (d.L) {
      case 4: launch_packed<uint8_t, 4>(p, batch, n_in, d, pk, n_out, out, vec, lif, s); break;
      case 5: launch_packed<uint8_t, 5>(p, batch, n_in, d, pk, n_out, out, vec, lif, s); break;
      default: launch_packed<uint8_t, 6>(p, batch, n_in, d, pk, n_out, out, vec, lif, s); break;
    }
  } else {
    const float* p = (const float*)spk;
    switch (d.L) {
      case 4: launch_packed<float, 4>(p, batch, n_in, d, pk, n_out, out, vec, lif, s); break;
      case 5: launch_packed<float, 5>(p, batch, n_in, d, pk, n_out, out, vec, lif, s); break;
      default: launch_packed<float, 6>(p, batch, n_in, d, pk, n_out, out, vec, lif, s); break;
    }
  }
  BS_CHECK_LAUNCH();
  return BS_OK;
}

}  // namespace

extern "C" int32_t bs_event_dense_digits(int32_t n_in) { return digits_for(n_in); }

extern "C" int64_t bs_event_dense_packed_bytes(int32_t n_in, int32_t n_out) {
  if (n_out < 0 || digits_for(n_in) == 0) return 0;
  return pack_dims(n_in, n_out).total;
}

extern "C" int bs_event_dense_pack(const float* W, int32_t n_in, int32_t n_out, void* packed,
                                   int64_t packed_bytes, bs_stream_t stream) {
  bs_clear_error();
  BS_CHECK_ARG(n_in >= 0 && n_out >= 0, "bs_event_dense_pack: negative size");
  BS_CHECK_ARG(n_in <= kMaxIn, "bs_event_dense_pack: n_in = %d exceeds %d", n_in, kMaxIn);
  const PackDims d = pack_dims(n_in, n_out);
  BS_CHECK_ARG(packed != nullptr && ((uintptr_t)packed & 255) == 0,
               "bs_event_dense_pack: packed buffer must be non-NULL and 256-byte aligned");
  BS_CHECK_ARG(packed_bytes >= d.total,
               "bs_event_dense_pack: packed buffer of %lld bytes needed (got %lld)",
               (long long)d.total, (long long)packed_bytes);
  BS_CHECK_ARG(W != nullptr || (int64_t)n_in * n_out == 0, "bs_event_dense_pack: W is NULL");
  hipStream_t s = bs_stream(stream);
  uint8_t* base = (uint8_t*)packed;
  uint32_t* status = (uint32_t*)base;
  uint32_t* bits = (uint32_t*)(base + d.bits_off);
  const int64_t clear_words = d.dig_off / 4;
  k_pack_clear<<<(int)((clear_words + 255) / 256), 256, 0, s>>>(status, clear_words);
  BS_CHECK_LAUNCH();
  if ((int64_t)n_in * n_out > 0) {
    const dim3 g((n_out + 63) / 64, (n_in + kMaxRowsWg - 1) / kMaxRowsWg);
    k_pack_colmax<<<g, 256, 0, s>>>(W, n_in, n_out, status, bits);
    BS_CHECK_LAUNCH();
  }
  const int64_t threads = (int64_t)d.NT * kTileN * d.KB * 4;
  if (threads > 0) {
    const int64_t blocks = (threads + 255) / 256;
    BS_CHECK_ARG(blocks <= INT32_MAX, "bs_event_dense_pack: W too large");
    uint8_t* dig = base + d.dig_off;
    switch (d.L) {
      case 4: k_pack_digits<4><<<(int)blocks, 256, 0, s>>>(W, n_in, n_out, d.KB, d.NT, bits, dig); break;
      case 5: k_pack_digits<5><<<(int)blocks, 256, 0, s>>>(W, n_in, n_out, d.KB, d.NT, bits, dig); break;
      default: k_pack_digits<6><<<(int)blocks, 256, 0, s>>>(W, n_in, n_out, d.KB, d.NT, bits, dig); break;
    }
    BS_CHECK_LAUNCH();
  }
  return BS_OK;
}

extern "C" int bs_event_dense_packed_f32(const void* spk, int32_t spk_dtype, int32_t batch,
                                         int32_t n_in, const void* packed, int32_t n_out,
                                         float* out, bs_stream_t stream) {
  bs_clear_error();
  return packed_product("bs_event_dense_packed_f32", spk, spk_dtype, batch, n_in, packed, n_out,
                        out, nullptr, bs_stream(stream));
}

extern "C" int bs_event_dense_packed_lif_step(const void* spk, int32_t spk_dtype, int32_t batch,
                                              int32_t n_in, const void* packed, int32_t n_out,
                                              int32_t inh, float* V, float* ge, float* gi,
                                              int32_t* ref, const bs_lif_params* p,
                                              float* cur_out, uint8_t* spk_out,
                                              bs_stream_t stream) {
  bs_clear_error();
  const char* fn = "bs_event_dense_packed_lif_step";
  BS_CHECK_ARG(p != nullptr, "%s: params are NULL", fn);
  BS_CHECK_ARG(!p->deferred_reset, "%s: deferred_reset is not supported by the fused step "
               "(use bs_event_dense_packed_f32 and bs_coba_lif_step)", fn);
  BS_CHECK_ARG((int64_t)batch * n_out <= 0 || (V && ge && gi && ref), "%s: NULL state pointer",
               fn);
  // Workgroups of other column tiles read the spikes of a batch row while one writes that
  // row's outputs, so no output may share memory with the spike input (a recurrent caller
  // passing one buffer as both would read spikes of this step).
  if ((int64_t)batch * n_in > 0 && (int64_t)batch * n_out > 0 && spk != nullptr) {
    const uintptr_t s0 = (uintptr_t)spk;
    const uintptr_t s1 = s0 + (uintptr_t)batch * n_in * (spk_dtype == BS_SPK_F32 ? 4 : 1);
    const uintptr_t no = (uintptr_t)batch * n_out;
    auto overlaps = [&](const void* q, uintptr_t bytes) {
      const uintptr_t q0 = (uintptr_t)q;
      return q != nullptr && q0 < s1 && s0 < q0 + bytes;
    };
    BS_CHECK_ARG(!overlaps(spk_out, no) && !overlaps(cur_out, 4 * no) && !overlaps(V, 4 * no) &&
                     !overlaps(ge, 4 * no) && !overlaps(gi, 4 * no) && !overlaps(ref, 4 * no),
                 "%s: an output (spk_out, cur_out or the neuron state) overlaps the spike input",
                 fn);
  }
  LifOut lif{V, ge, gi, ref, spk_out, inh ? 1 : 0, *p};
  return packed_product(fn, spk, spk_dtype, batch, n_in, packed, n_out, cur_out, &lif,
                        bs_stream(stream));
}

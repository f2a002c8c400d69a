// Speculative-sampling acceptance and row sampling over the full vocabulary (gfx950).
//
// Semantics follow src/generate.py:17-37 (temperature, top-k keeping every token
// >= the k-th largest logit, top-p keeping a token iff the mass ranked strictly
// above it is <= top_p, greedy argmax at T <= 0) plus the rejection rule on top of
// src/qwen3_5/mtp.py:144-155: accept draft d at position i iff u q_i(d) < p_i(d); at
// the first rejection draw from norm(max(0, p_i - q_i)); if every draft is accepted
// draw the bonus token from p_k.
//
// The arithmetic is specified so that it has no reduction-order freedom:
//   sampling key    bf16 logit with |x| <= 2^-16 flushed to 0; equal keys are ties
//   weight          w = trunc(2^39 * 2^((x - x_max) * inv_T * log2 e)), with 2^t
//                   evaluated as 2^n * P(f) (Cody-Waite split, degree-7 Taylor of
//                   2^f on [-1/2, 1/2], fmaf Horner); zero below t = -40 and for
//                   tokens more than NBINS keys under the maximum
//   every mass      an exact unsigned integer sum (u64, u128 for residuals)
//   uniforms        Philox4x32-10, key (seed lo, hi), counter (row, offset lo, hi,
//                   slot / 4), word slot % 4, U = word >> 8
// so any parallel decomposition gives the same bits.  This file is compiled with
// -ffp-contract=off.
//
// Kernels:
//   row_stats    one 1024-thread workgroup per row (target and draft rows in one
//                launch), two per CU (64 registers per thread), one HBM pass: the first
//                8 x 16 B per thread of the row stay in registers and give a lower bound
//                of the max key; the whole row is counted as it streams into a per-key
//                histogram in LDS over a window of 2 NBINS keys ending NBINS above that
//                bound (distances computed two tokens at a time in packed 16-bit
//                arithmetic), which holds the NBINS keys below the row's max key
//                whenever the max lies within NBINS keys of the bound (otherwise the row
//                is counted again); then block scans for the top-k / top-p cut points
//                and the kept mass Z;
//   row_stats_known  the same for rows whose max key is given (the verify lm_head's
//                row-maximum slots): the whole row in registers, counted directly;
//   argmax_*     greedy rows: the row split over 16 workgroups, partial maxima
//                merged by a second tiny kernel (a greedy row needs no histogram);
//   spec_partial / spec_final  the k accept tests in parallel, then the residual or
//                bonus draw in two passes: ns workgroups per sequence sum the draw's
//                weights over ns contiguous vocabulary slices, then one workgroup per
//                sequence locates the slice holding the target and the token in it;
//   sample_rows  one draw per row.
// A draw is an inverse CDF over token ids in three steps: every wave of the block sums
// the weights of its own contiguous sixteenth of the range (coalesced, exact integers,
// the next 2-4 chunks per lane in flight), the sixteenth holding the target is summed
// again split over the 16 waves, and the one wave whose part holds the target walks it
// with wave-level scans.  A token's weight depends only on its key's distance below the
// row maximum (computed two tokens at a time in packed 16-bit arithmetic), so each draw
// first fills an LDS table of the weights of the distances within the cut (the same
// weight_of) and reads an entry only for tokens within the cut.  Residual masses are 64-bit when q is
// one-hot (argmax drafts) and 128-bit when q is a sampled distribution.
#include "common.h"

#include <algorithm>
#include <mutex>

namespace lollm {

typedef unsigned __int128 u128;

constexpr int SP_THREADS = 1024;
constexpr int SP_NBINS = 8192;
constexpr int SP_MAG0 = 0x3780;  // bf16 magnitude of 2^-16

struct RowStat {
  int32_t argmax, kmax, cut, greedy;
  uint64_t Z;
};

// ---------------------------------------------------------------- Philox4x32-10
__device__ __forceinline__ uint32_t philox_u24(uint64_t seed, uint64_t offset, uint32_t row,
                                               uint32_t slot) {
  uint32_t c0 = row, c1 = (uint32_t)offset, c2 = (uint32_t)(offset >> 32), c3 = slot >> 2;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
  }
  const uint32_t w[4] = {c0, c1, c2, c3};
  return w[slot & 3] >> 8;
}

// ---------------------------------------------------------------- keys and weights
__device__ __forceinline__ int32_t skey(uint32_t b) {
  const int32_t mag = b & 0x7FFF;
  const int32_t mc = mag > SP_MAG0 ? mag - SP_MAG0 : 0;
  return (b & 0x8000) ? -mc : mc;
}

__device__ __forceinline__ float key_value(int32_t key) {
  if (key == 0) return 0.0f;
  const uint32_t mag = (uint32_t)(key > 0 ? key : -key) + SP_MAG0;
  return __uint_as_float((mag | (key < 0 ? 0x8000u : 0u)) << 16);
}

__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  return (b & 0x8000) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

__device__ __forceinline__ float spec_exp2(float t) {
  const float c1 = 0.693147180559945309f, c2 = 0.240226506959100712f,
              c3 = 0.0555041086648215800f, c4 = 0.00961812910762847717f,
              c5 = 0.00133335581464284434f, c6 = 1.54035303933816099e-4f,
              c7 = 1.52527338040598403e-5f;
  const float n = __builtin_rintf(t);
  const float f = t - n;
  float p = c7;
  p = __builtin_fmaf(p, f, c6);
  p = __builtin_fmaf(p, f, c5);
  p = __builtin_fmaf(p, f, c4);
  p = __builtin_fmaf(p, f, c3);
  p = __builtin_fmaf(p, f, c2);
  p = __builtin_fmaf(p, f, c1);
  p = __builtin_fmaf(p, f, 1.0f);
  return __builtin_amdgcn_ldexpf(p, (int)n);
}

__device__ __forceinline__ uint64_t weight_of(float x, float xmax, float c) {
  const float t = (x - xmax) * c;
  if (!(t >= -40.0f)) return 0;
  const float e = spec_exp2(t);
  return (uint64_t)(e * 549755813888.0f);  // 2^39
}

__device__ __forceinline__ uint64_t token_weight(const RowStat& s, float c, uint32_t b,
                                                 int32_t tok) {
  if (s.greedy) return tok == s.argmax ? 1u : 0u;
  const int32_t k = skey(b);
  if (s.kmax - k > s.cut) return 0;
  return weight_of(key_value(k), key_value(s.kmax), c);
}

// Weight table of a row's distribution: tab[d] = the weight of a token whose key is d
// below the row's maximum key, filled for d <= cut only (the only entries read).
__device__ void build_table(const RowStat& s, float c, uint64_t* tab) {
  if (s.greedy) return;
  const float xmax = key_value(s.kmax);
  for (int d = threadIdx.x; d <= s.cut; d += blockDim.x)
    tab[d] = weight_of(key_value(s.kmax - d), xmax, c);
}

// Order keys of the two bf16 in a word, packed (ord16 per half).
__device__ __forceinline__ uint32_t ord_pair(uint32_t w) {
  const uint32_t sgn = (w >> 15) & 0x00010001u;
  return w ^ ((sgn * 0x7FFFu) | 0x80008000u);
}

typedef unsigned short sp_us2 __attribute__((ext_vector_type(2)));
typedef short sp_s2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(sp_us2, a),
                                                                __builtin_bit_cast(sp_us2, b)));
}

// Distances below the row's maximum key, kmax - skey(b), of the two bf16 of w as 16-bit
// halves (every bf16 pattern gives a distance in [0, 2^16)).  km2 holds kmax mod 2^16 in
// both halves.  With s = 0 / -1 the sign mask and m = max(|b| - SP_MAG0, 0):
// skey = s ? -m : m, so kmax - skey = (kmax + s) - (m ^ s) modulo 2^16.
__device__ __forceinline__ uint32_t dist_pair(uint32_t w, uint32_t km2) {
  const sp_us2 s = __builtin_bit_cast(sp_us2, __builtin_bit_cast(sp_s2, w) >> (short)15);
  const sp_us2 mag = __builtin_bit_cast(sp_us2, w & 0x7FFF7FFFu);
  const sp_us2 m = __builtin_elementwise_sub_sat(mag, (sp_us2)((unsigned short)SP_MAG0));
  const sp_us2 d = (__builtin_bit_cast(sp_us2, km2) + s) - (m ^ s);
  return __builtin_bit_cast(uint32_t, d);
}

// The weights of the two tokens of word w (tokens t0, t0 + 1) under a row's distribution
// (token_weight as a lookup): the table entry of each token's distance below the
// maximum, read only for distances within the cut (every other token weighs 0).
__device__ __forceinline__ void pair_weights(const RowStat& s, const uint64_t* tab, uint32_t w,
                                             int t0, uint64_t& w0, uint64_t& w1) {
  if (s.greedy) {
    w0 = t0 == s.argmax ? 1u : 0u;
    w1 = t0 + 1 == s.argmax ? 1u : 0u;
    return;
  }
  const uint32_t dd = dist_pair(w, ((uint32_t)s.kmax & 0xFFFFu) * 0x10001u);
  const int32_t d0 = (int32_t)(dd & 0xFFFFu), d1 = (int32_t)(dd >> 16);
  w0 = d0 <= s.cut ? tab[d0] : 0;
  w1 = d1 <= s.cut ? tab[d1] : 0;
}

__device__ __forceinline__ void chunk_weights(const RowStat& s, const uint64_t* tab,
                                              const u32x4_t& u, int ch, uint64_t* w) {
  pair_weights(s, tab, u.x, ch * 8, w[0], w[1]);
  pair_weights(s, tab, u.y, ch * 8 + 2, w[2], w[3]);
  pair_weights(s, tab, u.z, ch * 8 + 4, w[4], w[5]);
  pair_weights(s, tab, u.w, ch * 8 + 6, w[6], w[7]);
}

// bf16 bits of an order key (inverse of ord16)
__device__ __forceinline__ uint32_t ord_bits(uint32_t o) {
  return (o & 0x8000u) ? (o ^ 0x8000u) : (~o & 0xFFFFu);
}

// ---------------------------------------------------------------- block primitives
template <typename T>
__device__ __forceinline__ T shfl_up_any(T v, int d) {
  constexpr int W = (sizeof(T) + 3) / 4;
  union { T v; uint32_t w[W]; } u, r;
  u.v = v;
#pragma unroll
  for (int i = 0; i < W; ++i) r.w[i] = __shfl_up(u.w[i], d, 64);
  return r.v;
}

template <typename T>
__device__ __forceinline__ T shfl_xor_any(T v, int m) {
  constexpr int W = (sizeof(T) + 3) / 4;
  union { T v; uint32_t w[W]; } u, r;
  u.v = v;
#pragma unroll
  for (int i = 0; i < W; ++i) r.w[i] = __shfl_xor(u.w[i], m, 64);
  return r.v;
}

// Inclusive scan over the block (exact for integers).  `scratch` holds 16 T.
template <typename T>
__device__ T block_inclusive_scan(T v, T* scratch, T* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    T o = shfl_up_any(v, d);
    if (lane >= d) v += o;
  }
  if (lane == 63) scratch[wave] = v;
  __syncthreads();
  T before = 0, all = 0;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) {
    const T s = scratch[w];
    if (w < wave) before += s;
    all += s;
  }
  __syncthreads();
  *total = all;
  return v + before;
}

template <typename T>
__device__ T block_sum(T v, T* scratch) {
  T total;
  block_inclusive_scan(v, scratch, &total);
  return total;
}

template <typename T>
__device__ T block_max(T v, T* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    T o = shfl_xor_any(v, m);
    v = o > v ? o : v;
  }
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  T r = scratch[0];
  const int nw = blockDim.x >> 6;
  for (int w = 1; w < nw; ++w) r = scratch[w] > r ? scratch[w] : r;
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------- block primitives
template <typename T>
__device__ __forceinline__ T wave_sum_any(T v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += shfl_xor_any(v, m);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T o = shfl_up_any(v, d);
    if (lane >= d) v += o;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ T shfl_any(T v, int src) {
  constexpr int W = (sizeof(T) + 3) / 4;
  union { T v; uint32_t w[W]; } u, r;
  u.v = v;
#pragma unroll
  for (int i = 0; i < W; ++i) r.w[i] = __shfl(u.w[i], src, 64);
  return r.v;
}

// ---------------------------------------------------------------- row statistics
constexpr int SP_REG = 8;        // 16-byte chunks per thread held in registers
constexpr int SP_TAIL = 4;       // chunks per thread in flight in each tail batch
constexpr int SP_NSPLIT = 16;    // workgroups per greedy row

__device__ __forceinline__ void scan_chunk(uint4 u, int c, uint64_t& best, int32_t& km) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t b = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
    const uint32_t idx = (uint32_t)(c * 8 + e);
    const uint64_t packed = ((uint64_t)ord16(b) << 32) | (0xFFFFFFFFu - idx);
    best = packed > best ? packed : best;
    const int32_t k = skey(b);
    km = k > km ? k : km;
  }
}

// Counts of the 8 tokens of a chunk by distance below the maximum key; only distances
// <= dlim (< SP_NBINS) are counted.
__device__ __forceinline__ void hist_chunk(uint4 u, uint32_t km2, int32_t dlim, uint32_t* hist) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t dd = dist_pair(w[h], km2);
    const int32_t d0 = (int32_t)(dd & 0xFFFFu), d1 = (int32_t)(dd >> 16);
    if (d0 <= dlim) atomicAdd(&hist[d0], 1u);
    if (d1 <= dlim) atomicAdd(&hist[d1], 1u);
  }
}

// The rest of a sampled row's statistics once its maximum is known (top_bits: the bf16
// bits of the largest logit): the distances that need counting, the per-key counts
// (count(km2, dlim) fills hist; km2 = the maximum key mod 2^16 in both halves), then
// block scans for the top-k / top-p cut points and the kept mass Z.  hist must be zero
// and visible to every thread before the call.
template <typename Count>
__device__ __forceinline__ void row_stats_counts(uint32_t top_bits, float inv_temp, int top_k,
                                                 float top_p, RowStat* out, uint32_t* hist,
                                                 uint64_t* s64, int32_t* shared_cut_p,
                                                 uint64_t* z_sh_p, Count count) {
  const int tid = threadIdx.x;
  int32_t& shared_cut = *shared_cut_p;
  uint64_t& z_sh = *z_sh_p;
  RowStat st;
  st.greedy = 0;
  st.argmax = -1;   // only greedy rows use it
  const int32_t km = skey(top_bits);
  st.kmax = km;
  const float xmax = key_value(km);
  const float c = inv_temp * 1.44269504088896341f;
  // ---- which distances need counting: all below SP_NBINS when top-k reads the counts;
  //      without top-k only the mass (count x weight) is read, so distances whose weight
  //      test t = (x - xmax) c >= -40 fails (weight 0) are skipped.  t does not increase
  //      with the distance, so those distances are a suffix: bisect for its start over
  //      the distances of real keys (skey >= -(0x7FFF - SP_MAG0)). ----
  int32_t dlim = SP_NBINS - 1;
  if (top_k <= 0) {
    if (!((xmax - xmax) * c >= -40.0f)) {
      dlim = -1;   // the maximum is inf or NaN: every weight is zero
    } else {
      int lo = 0, hi = min(SP_NBINS - 1, km + (0x7FFF - SP_MAG0)) + 1;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if ((key_value(km - mid) - xmax) * c >= -40.0f) lo = mid; else hi = mid;
      }
      dlim = lo;
    }
  }
  // ---- per-key counts below the max ----
  const uint32_t km2 = ((uint32_t)km & 0xFFFFu) * 0x10001u;
  count(km2, dlim);
  __syncthreads();
  // ---- cut points and kept mass: thread t owns bins [8t, 8t + 8) ----
  constexpr int PER = SP_NBINS / SP_THREADS;
  uint32_t cnt[PER];
  uint64_t mass[PER];
  uint32_t csum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int d = tid * PER + j;
    cnt[j] = hist[d];
    mass[j] = cnt[j] ? (uint64_t)cnt[j] * weight_of(key_value(km - d), xmax, c) : 0;
    csum += cnt[j];
  }
  if (tid == 0) shared_cut = SP_NBINS - 1;
  __syncthreads();
  if (top_k > 0) {
    uint64_t ctot;
    const uint64_t cinc = block_inclusive_scan<uint64_t>((uint64_t)csum, s64, &ctot);
    const uint64_t c0 = cinc - csum;
    if (c0 < (uint64_t)top_k && cinc >= (uint64_t)top_k) {
      uint64_t run = c0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        run += cnt[j];
        if (run >= (uint64_t)top_k) { shared_cut = tid * PER + j; break; }
      }
    }
    __syncthreads();
  }
  const int32_t cut_k = shared_cut;
  uint64_t msum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (tid * PER + j <= cut_k) msum += mass[j];
  uint64_t W;
  const uint64_t minc = block_inclusive_scan<uint64_t>(msum, s64, &W);
  st.cut = cut_k;
  st.Z = W;
  if (top_p > 0.0f && top_p < 1.0f) {
    const uint32_t p24 = (uint32_t)(top_p * 16777216.0f);
    const uint64_t tm = (uint64_t)(((u128)W * p24) >> 24);
    const uint64_t m0 = minc - msum;
    if (m0 <= tm && minc > tm) {
      uint64_t run = m0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        if (tid * PER + j > cut_k) break;
        run += mass[j];
        if (run > tm) { shared_cut = tid * PER + j; z_sh = run; break; }
      }
    }
    __syncthreads();
    st.cut = shared_cut;
    st.Z = z_sh;
  }
  if (tid == 0) *out = st;
}


// Sampled rows only (inv_temp > 0); greedy rows take the split argmax below.  Rows
// [0, rows0) are read from x0, the rest from x1 (target and draft rows in one launch).
// One HBM pass: the maximum is not known while the row streams, so the keys are
// counted into a window of SP_WIN keys that ends SP_NBINS keys above the maximum of
// the first SP_REG chunks per thread (a lower bound of the row's maximum km); any
// maximum up to that end leaves every distance 0 .. SP_NBINS - 1 below km inside the
// window, so the histogram of row_stats_counts is the window from (end - km) on.  A row
// whose maximum lies further above is read and counted again in a zeroed window.
// Without top-k every key in the window is counted (the counts whose weight test fails
// weigh 0 in the mass and are read for nothing else).
constexpr int SP_WIN = 2 * SP_NBINS;

// The order-key maximum of a chunk's 8 tokens, folded into m2 (two 16-bit halves).
__device__ __forceinline__ uint32_t ord_max_chunk(uint32_t m2, const uint4& u) {
  return max_u16x2(max_u16x2(m2, ord_pair(u.x)),
                   max_u16x2(max_u16x2(ord_pair(u.y), ord_pair(u.z)), ord_pair(u.w)));
}

__global__ __launch_bounds__(SP_THREADS, 8) void row_stats_kernel(const uint16_t* __restrict__ x0,
                                                               int rows0,
                                                               const uint16_t* __restrict__ x1,
                                                               int V, float inv_temp, int top_k,
                                                               float top_p, RowStat* stats) {
  __shared__ uint32_t win[SP_WIN];
  __shared__ uint64_t s64[16];
  __shared__ int32_t shared_cut;
  __shared__ uint64_t z_sh;
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int nch = V >> 3;
  const uint16_t* src = row < rows0 ? x0 + (size_t)row * V : x1 + (size_t)(row - rows0) * V;
  const uint4* x4 = reinterpret_cast<const uint4*>(src);
  // ---- the first SP_REG chunks per thread into registers; zero the window meanwhile ----
  uint4 reg[SP_REG];
#pragma unroll
  for (int i = 0; i < SP_REG; ++i) reg[i] = x4[min(i * SP_THREADS + tid, nch - 1)];
  for (int i = tid; i < SP_WIN; i += SP_THREADS) win[i] = 0u;
  uint32_t m2 = 0;   // order keys: 0 is below every token's
#pragma unroll
  for (int i = 0; i < SP_REG; ++i)
    if (i * SP_THREADS + tid < nch) m2 = ord_max_chunk(m2, reg[i]);
  // the window's end (block_max's barriers also publish the zeroed window)
  const int32_t k0 =
      skey(ord_bits((uint32_t)block_max<uint64_t>((uint64_t)max(m2 & 0xFFFFu, m2 >> 16), s64)));
  const int32_t kend = k0 + SP_NBINS;
  const uint32_t ke2 = ((uint32_t)kend & 0xFFFFu) * 0x10001u;
#pragma unroll
  for (int i = 0; i < SP_REG; ++i)
    if (i * SP_THREADS + tid < nch) hist_chunk(reg[i], ke2, SP_WIN - 1, win);
  // the rest of the row in batches, counted as it arrives (addresses clamped into the
  // row; the repeats are neither counted nor maximised)
  for (int c0 = SP_REG * SP_THREADS + tid; c0 < nch; c0 += SP_TAIL * SP_THREADS) {
    uint4 tl[SP_TAIL];
#pragma unroll
    for (int u = 0; u < SP_TAIL; ++u) tl[u] = x4[min(c0 + u * SP_THREADS, nch - 1)];
#pragma unroll
    for (int u = 0; u < SP_TAIL; ++u)
      if (c0 + u * SP_THREADS < nch) {
        m2 = ord_max_chunk(m2, tl[u]);
        hist_chunk(tl[u], ke2, SP_WIN - 1, win);
      }
  }
  const uint32_t top_bits =
      ord_bits((uint32_t)block_max<uint64_t>((uint64_t)max(m2 & 0xFFFFu, m2 >> 16), s64));
  const int32_t km = skey(top_bits);
  const bool inside = km <= kend;   // the same in every thread
  row_stats_counts(top_bits, inv_temp, top_k, top_p, stats + row, inside ? win + (kend - km) : win,
                   s64, &shared_cut, &z_sh, [&](uint32_t km2, int32_t dlim) {
    if (inside) return;
    // the maximum lies above the window: count the whole row again below km
    __syncthreads();
    for (int i = tid; i < SP_NBINS; i += SP_THREADS) win[i] = 0u;
    __syncthreads();
    for (int c0 = tid; c0 < nch; c0 += SP_TAIL * SP_THREADS) {
      uint4 tl[SP_TAIL];
#pragma unroll
      for (int u = 0; u < SP_TAIL; ++u) tl[u] = x4[min(c0 + u * SP_THREADS, nch - 1)];
#pragma unroll
      for (int u = 0; u < SP_TAIL; ++u)
        if (c0 + u * SP_THREADS < nch) hist_chunk(tl[u], km2, dlim, win);
    }
  });
}

// Sampled rows whose maxima are given: row r's maximum order key is the largest of
// rmax[r * rmax_ld + 0 .. rmax_slots) (the row-maximum slots of lollm_gemm_logits), so
// the row is read once, straight into the counts: no maximum pass and no second read of
// the row.  One workgroup per CU (128 registers per thread): the first SP_KREG 16-byte
// chunks per thread -- the whole row at V <= 163840 -- are requested together, so a row
// costs one memory round trip; any rest follows in batches.
constexpr int SP_KREG = 20;

__global__ __launch_bounds__(SP_THREADS, 4) void row_stats_known_kernel(
    const uint16_t* __restrict__ x, int V, float inv_temp, int top_k, float top_p,
    RowStat* stats, const uint16_t* __restrict__ rmax, long long rmax_ld, int rmax_slots) {
  __shared__ uint32_t hist[SP_NBINS];
  __shared__ uint64_t s64[16];
  __shared__ int32_t shared_cut;
  __shared__ uint64_t z_sh;
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int nch = V >> 3;
  const uint4* x4 = reinterpret_cast<const uint4*>(x + (size_t)row * V);
  uint4 reg[SP_KREG];
#pragma unroll
  for (int i = 0; i < SP_KREG; ++i) reg[i] = x4[min(i * SP_THREADS + tid, nch - 1)];
  uint32_t mo = 0;
  for (int i = tid; i < rmax_slots; i += SP_THREADS) mo = max(mo, (uint32_t)rmax[(size_t)row * rmax_ld + i]);
  for (int i = tid; i < SP_NBINS; i += SP_THREADS) hist[i] = 0;
  const uint32_t top_bits = ord_bits((uint32_t)block_max<uint64_t>((uint64_t)mo, s64));
  row_stats_counts(top_bits, inv_temp, top_k, top_p, stats + row, hist, s64, &shared_cut, &z_sh,
                   [&](uint32_t km2, int32_t dlim) {
#pragma unroll
    for (int i = 0; i < SP_KREG; ++i)
      if (i * SP_THREADS + tid < nch) hist_chunk(reg[i], km2, dlim, hist);
    for (int c0 = SP_KREG * SP_THREADS + tid; c0 < nch; c0 += SP_TAIL * SP_THREADS) {
      uint4 tl[SP_TAIL];
#pragma unroll
      for (int u = 0; u < SP_TAIL; ++u) tl[u] = x4[min(c0 + u * SP_THREADS, nch - 1)];
#pragma unroll
      for (int u = 0; u < SP_TAIL; ++u)
        if (c0 + u * SP_THREADS < nch) hist_chunk(tl[u], km2, dlim, hist);
    }
  });
}

// Greedy rows: 16 workgroups per row each reduce a slice to a packed
// (order key, ~index) maximum; a second kernel merges them into RowStat / a token.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const uint16_t* __restrict__ logits,
                                                             int V, uint64_t* __restrict__ part) {
  __shared__ uint64_t s64[4];
  const int row = blockIdx.y, split = blockIdx.x;
  const int nch = V >> 3, per = (nch + SP_NSPLIT - 1) / SP_NSPLIT;
  const int c0 = split * per, c1 = min(nch, c0 + per);
  const uint4* x4 = reinterpret_cast<const uint4*>(logits + (size_t)row * V);
  uint64_t best = 0;
  int32_t km = 0;
  for (int c = c0 + threadIdx.x; c < c1; c += 256) scan_chunk(x4[c], c, best, km);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint64_t o = shfl_xor_any(best, m);
    best = o > best ? o : best;
  }
  if (lane == 0) s64[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t r = s64[0];
    for (int w = 1; w < 4; ++w) r = s64[w] > r ? s64[w] : r;
    part[(size_t)row * SP_NSPLIT + split] = r;
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const uint64_t* __restrict__ part,
                                                          RowStat* __restrict__ stats,
                                                          int32_t* __restrict__ tokens) {
  const int row = blockIdx.x, lane = threadIdx.x;
  uint64_t best = lane < SP_NSPLIT ? part[(size_t)row * SP_NSPLIT + lane] : 0;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint64_t o = shfl_xor_any(best, m);
    best = o > best ? o : best;
  }
  if (lane == 0) {
    const int32_t am = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
    if (stats) {
      RowStat st;
      st.argmax = am; st.kmax = 0; st.cut = 0; st.greedy = 1; st.Z = 1;
      stats[row] = st;
    }
    if (tokens) tokens[row] = am;
  }
}

// ---------------------------------------------------------------- inverse-CDF draw
// Over the chunk range [lo, hi), wave w of the 16 owns [lo + w seg, min(lo + (w + 1) seg,
// hi)) with seg = ceil((hi - lo) / 16).  ld(c) loads chunk c (8 tokens; addresses stay in
// [lo, hi)), wt(raw, c, w[8]) turns it into the 8 token weights.
__device__ __forceinline__ int range_seg(int lo, int hi) {
  return (hi - lo + SP_THREADS / 64 - 1) / (SP_THREADS / 64);
}

// Per-wave totals of [lo, hi) into wtot[16]; returns the range total.  Every lane loads
// UN chunks at a time (unconditionally, at clamped addresses) before it sums them.
template <typename Acc, int UN, typename LD, typename WT>
__device__ Acc draw_totals(int lo, int hi, LD ld, WT wt, Acc* wtot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // wtot may still be read by a previous draw's waves
  const int seg = range_seg(lo, hi);
  const int c0 = lo + wave * seg, c1 = min(c0 + seg, hi);
  Acc acc = 0;
  for (int cb = c0; cb < c1; cb += 64 * UN) {
    decltype(ld(0)) r[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) r[u] = ld(min(cb + lane + 64 * u, c1 - 1));
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int c = cb + lane + 64 * u;
      Acc w[8];
      wt(r[u], c, w);
      Acc s = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) s += w[e];
      acc += c < c1 ? s : (Acc)0;
    }
  }
  acc = wave_sum_any(acc);
  if (lane == 0) wtot[wave] = acc;
  __syncthreads();
  Acc tot = 0;
#pragma unroll
  for (int w = 0; w < SP_THREADS / 64; ++w) tot += wtot[w];
  return tot;
}

// The first token of [lo, hi) whose inclusive prefix (from lo) exceeds target (< the
// range total held in wtot by draw_totals).
template <typename Acc, typename LD, typename WT>
__device__ int32_t draw_find(int lo, int hi, LD ld, WT wt, const Acc* wtot, Acc target, int V,
                             int32_t* found) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Acc before = 0;
  int ow = SP_THREADS / 64 - 1;
  for (int w = 0; w < SP_THREADS / 64; ++w) {
    if (before + wtot[w] > target) { ow = w; break; }
    before += wtot[w];
  }
  if (threadIdx.x == 0) *found = -1;
  __syncthreads();
  const int seg = range_seg(lo, hi);
  const int c0 = lo + ow * seg, c1 = min(c0 + seg, hi);
  if (wave == ow && c0 < c1) {
    Acc run = before;
    auto cur = ld(min(c0 + lane, c1 - 1));
    for (int cb = c0; cb < c1; cb += 64) {
      const int c = cb + lane;
      const auto nxt = ld(min(cb + 64 + lane, c1 - 1));   // next step's chunk, in flight
      Acc w[8];
      Acc sum = 0;
      if (c < c1) {
        wt(cur, c, w);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = 0;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += w[e];
      const Acc inc = wave_incl_scan(sum);
      const Acc tot = shfl_any(inc, 63);
      if (run + tot > target) {
        const Acc ex = run + inc - sum;
        if (ex <= target && run + inc > target) {
          Acc r = ex;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            r += w[e];
            if (r > target) { *found = c * 8 + e; break; }
          }
        }
        break;
      }
      run += tot;
      cur = nxt;
    }
  }
  __syncthreads();
  const int32_t f = *found;
  return f < 0 ? V - 1 : f;
}

// The token at target in [lo, hi), given the per-wave totals draw_totals(lo, hi) left in
// wtot: for wave segments over two wave steps long, the segment that holds the target is
// summed again by all 16 waves first, so draw_find walks a sixteenth of it (1/256 of the
// range).
template <typename Acc, typename LD, typename WT>
__device__ int32_t draw_refine(int lo, int hi, LD ld, WT wt, Acc* wtot, Acc target, int V,
                               int32_t* found) {
  // a sixteenth of at most two wave steps is walked directly
  if (range_seg(lo, hi) <= 128) return draw_find<Acc>(lo, hi, ld, wt, wtot, target, V, found);
  Acc before = 0;
  int ow = SP_THREADS / 64 - 1;
  for (int w = 0; w < SP_THREADS / 64; ++w) {
    if (before + wtot[w] > target) { ow = w; break; }
    before += wtot[w];
  }
  const int seg = range_seg(lo, hi);
  const int lo1 = min(hi, lo + ow * seg), hi1 = min(lo1 + seg, hi);
  draw_totals<Acc, 1>(lo1, hi1, ld, wt, wtot);
  return draw_find<Acc>(lo1, hi1, ld, wt, wtot, target - before, V, found);
}

struct ChunkPair { u32x4_t p, q; };   // vector members: copies stay in registers

// chunks in flight per lane in the totals passes (64-bit and 128-bit masses)
constexpr int SP_UN64 = 4, SP_UN128 = 2;

__device__ __forceinline__ u128 scaled_target(uint32_t U, u128 M) {
  return (u128)U * (M >> 24) + (((u128)U * (uint64_t)(M & 0xFFFFFFu)) >> 24);
}

// Plain draw from a row's own distribution p (u64 masses, target floor(U Z / 2^24));
// tab is p's weight table (build_table), complete before the call.  REFINE: sum the
// sixteenth holding the target again before the walk (whole-row draws).
template <bool REFINE>
__device__ int32_t draw_plain(const uint16_t* xp, const RowStat& sp, const uint64_t* tab, uint32_t U,
                              int V, uint64_t* wtot, int32_t* found) {
  if (sp.greedy) return sp.argmax;
  const int nch = V >> 3;
  const u32x4_t* v4 = reinterpret_cast<const u32x4_t*>(xp);
  auto ld = [=](int ch) { return v4[ch]; };
  auto wt = [=](const u32x4_t& u, int ch, uint64_t* w) { chunk_weights(sp, tab, u, ch, w); };
  draw_totals<uint64_t, SP_UN64>(0, nch, ld, wt, wtot);
  const uint64_t tgt = (uint64_t)(((u128)U * sp.Z) >> 24);
  if constexpr (REFINE) return draw_refine<uint64_t>(0, nch, ld, wt, wtot, tgt, V, found);
  return draw_find<uint64_t>(0, nch, ld, wt, wtot, tgt, V, found);
}

// ---------------------------------------------------------------- acceptance
// The accept tests of sequence b (rows st_t[b (k+1) + i], st_d[b k + i]) and the
// distribution its emitted token is drawn from; every workgroup working on b derives
// the same plan.
struct AcceptPlan {
  int a;          // accepted drafts
  int kind;       // 0: p of row a (bonus, a == k), 1: residual with sampled q, 2: residual with one-hot q
  int d;          // the rejected draft (kinds 1, 2)
  uint32_t U;     // the draw's uniform
};

__device__ AcceptPlan accept_plan(const uint16_t* target, const uint16_t* draft,
                                  const int32_t* drafts, int k, int V, float c, uint64_t seed,
                                  uint64_t offset, const RowStat* st_t, const RowStat* st_d, int b,
                                  int32_t* ok) {
  for (int i = threadIdx.x; i < k; i += SP_THREADS) {
    int32_t d = drafts[b * k + i];
    d = d < 0 ? 0 : (d >= V ? V - 1 : d);
    const RowStat sp = st_t[b * (k + 1) + i];
    const uint16_t* xp = target + ((size_t)b * (k + 1) + i) * V;
    const uint64_t wp = token_weight(sp, c, xp[d], d), Zp = sp.Z;
    uint64_t wq = 1, Zq = 1;
    if (draft) {
      const RowStat sq = st_d[b * k + i];
      wq = token_weight(sq, c, draft[((size_t)b * k + i) * V + d], d);
      Zq = sq.Z;
    }
    const uint32_t Ui = philox_u24(seed, offset, (uint32_t)b, (uint32_t)i);
    const u128 lhs = (u128)Ui * wq * Zp;
    const u128 rhs = ((u128)wp * Zq) << 24;
    if (i < 64) ok[i] = lhs < rhs;
  }
  __syncthreads();
  AcceptPlan pl;
  pl.a = 0;
  while (pl.a < k && pl.a < 64 && ok[pl.a]) ++pl.a;
  pl.kind = pl.a == k ? 0 : (draft ? 1 : 2);
  int32_t d = pl.a < k ? drafts[b * k + pl.a] : 0;
  pl.d = d < 0 ? 0 : (d >= V ? V - 1 : d);
  pl.U = philox_u24(seed, offset, (uint32_t)b, (uint32_t)k);
  // the same in every lane (read from LDS after the barrier): make that visible to the
  // compiler so the plan, and the rows it selects, live in scalar registers
  pl.a = __builtin_amdgcn_readfirstlane(pl.a);
  pl.kind = __builtin_amdgcn_readfirstlane(pl.kind);
  pl.d = __builtin_amdgcn_readfirstlane(pl.d);
  pl.U = (uint32_t)__builtin_amdgcn_readfirstlane((int)pl.U);
  return pl;
}

// Runs f(ld, wt, acc_tag) with the chunk loader and weight function of the plan's draw
// (tables filled and visible on return from the setup).
template <typename F>
__device__ void with_draw(const AcceptPlan& pl, const uint16_t* target, const uint16_t* draft,
                          int k, int V, float c, const RowStat* st_t, const RowStat* st_d, int b,
                          uint64_t* tab_p, uint64_t* tab_q, F f) {
  const RowStat sp = st_t[b * (k + 1) + pl.a];
  const uint16_t* xp = target + ((size_t)b * (k + 1) + pl.a) * V;
  const u32x4_t* vp = reinterpret_cast<const u32x4_t*>(xp);
  build_table(sp, c, tab_p);
  if (pl.kind == 1) {
    // q a sampled distribution: residual wp Zq - wq Zp in 128 bits
    const RowStat sq = st_d[b * k + pl.a];
    const u32x4_t* vq = reinterpret_cast<const u32x4_t*>(draft + ((size_t)b * k + pl.a) * V);
    const uint64_t Zq = sq.Z;
    build_table(sq, c, tab_q);
    __syncthreads();
    auto ld = [=](int ch) { return ChunkPair{vp[ch], vq[ch]}; };
    auto wt = [=](const ChunkPair& r, int ch, u128* w) {
      const uint32_t pw[4] = {r.p.x, r.p.y, r.p.z, r.p.w}, qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        uint64_t wp[2], wq[2];
        pair_weights(sp, tab_p, pw[h], ch * 8 + 2 * h, wp[0], wp[1]);
        pair_weights(sq, tab_q, qw[h], ch * 8 + 2 * h, wq[0], wq[1]);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          u128 v = 0;
          if (wp[e] != 0) {   // most tokens lie past p's cut: skip the 128-bit products
            const u128 l = (u128)wp[e] * Zq, rr = (u128)wq[e] * sp.Z;
            v = l > rr ? l - rr : (u128)0;
          }
          w[2 * h + e] = v;
        }
      }
    };
    f(ld, wt, (u128)0);
  } else if (pl.kind == 2) {
    // q one-hot at d: residual wp - [t == d] Zp fits 64 bits
    __syncthreads();
    const int d = pl.d;
    auto ld = [=](int ch) { return vp[ch]; };
    auto wt = [=](const u32x4_t& up, int ch, uint64_t* w) {
      uint64_t wp[8];
      chunk_weights(sp, tab_p, up, ch, wp);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint64_t r = ch * 8 + e == d ? sp.Z : 0;
        w[e] = wp[e] > r ? wp[e] - r : 0;
      }
    };
    f(ld, wt, (uint64_t)0);
  } else {
    // the bonus: p of row k itself
    __syncthreads();
    auto ld = [=](int ch) { return vp[ch]; };
    auto wt = [=](const u32x4_t& u, int ch, uint64_t* w) { chunk_weights(sp, tab_p, u, ch, w); };
    f(ld, wt, (uint64_t)0);
  }
}

__device__ __forceinline__ void split_range(int nch, int ns, int s, int& lo, int& hi) {
  const int per = (nch + ns - 1) / ns;
  lo = min(nch, s * per);
  hi = min(nch, lo + per);
}

// Pass 1, grid (ns, B): workgroup (s, b) sums the draw's weights over the s-th of ns
// contiguous slices of the vocabulary, per wave: the 16 wave segments' exact totals
// (u128) in part[(b ns + s) 16 + w].
__global__ __launch_bounds__(SP_THREADS) void spec_partial_kernel(
    const uint16_t* __restrict__ target, const uint16_t* __restrict__ draft,
    const int32_t* __restrict__ drafts, int k, int V, float inv_temp, uint64_t seed,
    uint64_t offset_arg, const uint64_t* __restrict__ offset_dev, const RowStat* __restrict__ st_t,
    const RowStat* __restrict__ st_d, int ns, u128* __restrict__ part) {
  __shared__ u128 wt128[SP_THREADS / 64];
  __shared__ uint64_t wt64[SP_THREADS / 64];
  __shared__ int32_t ok[64];
  extern __shared__ uint64_t sp_tabs[];   // p's table, then q's when drafts are sampled
  uint64_t* tab_p = sp_tabs;
  uint64_t* tab_q = sp_tabs + SP_NBINS;
  const int s = blockIdx.x, b = blockIdx.y;
  const uint64_t offset = offset_dev ? *offset_dev : offset_arg;
  const float c = inv_temp * 1.44269504088896341f;
  const AcceptPlan pl = accept_plan(target, draft, drafts, k, V, c, seed, offset, st_t, st_d, b, ok);
  int lo, hi;
  split_range(V >> 3, ns, s, lo, hi);
  with_draw(pl, target, draft, k, V, c, st_t, st_d, b, tab_p, tab_q, [&](auto ld, auto wt, auto tag) {
    using Acc = decltype(tag);
    Acc* wtot;
    if constexpr (sizeof(Acc) == 16) wtot = wt128; else wtot = wt64;
    draw_totals<Acc, sizeof(Acc) == 16 ? SP_UN128 : SP_UN64>(lo, hi, ld, wt, wtot);
    if (threadIdx.x < SP_THREADS / 64)
      part[((size_t)b * ns + s) * (SP_THREADS / 64) + threadIdx.x] = (u128)wtot[threadIdx.x];
  });
}

// Pass 2, grid (B): the wave segment of pass 1 holding the target (from its totals), that
// segment summed again split over the 16 waves, and the owning sixteenth walked -- the
// same token as walking the whole slice, one pass over the slice fewer.
__global__ __launch_bounds__(SP_THREADS) void spec_final_kernel(
    const uint16_t* __restrict__ target, const uint16_t* __restrict__ draft,
    const int32_t* __restrict__ drafts, int k, int V, float inv_temp, uint64_t seed,
    uint64_t offset_arg, const uint64_t* __restrict__ offset_dev, const RowStat* __restrict__ st_t,
    const RowStat* __restrict__ st_d, int ns, const u128* __restrict__ part,
    int32_t* __restrict__ n_accepted, int32_t* __restrict__ next_token) {
  __shared__ u128 wt128[SP_THREADS / 64];
  __shared__ uint64_t wt64[SP_THREADS / 64];
  __shared__ int32_t found;
  __shared__ int32_t ok[64];
  extern __shared__ uint64_t sp_tabs[];
  uint64_t* tab_p = sp_tabs;
  uint64_t* tab_q = sp_tabs + SP_NBINS;
  const int b = blockIdx.x;
  const uint64_t offset = offset_dev ? *offset_dev : offset_arg;
  const float c = inv_temp * 1.44269504088896341f;
  const AcceptPlan pl = accept_plan(target, draft, drafts, k, V, c, seed, offset, st_t, st_d, b, ok);
  const RowStat sp = st_t[b * (k + 1) + pl.a];
  const int nch = V >> 3;
  constexpr int NW = SP_THREADS / 64;
  // the ns x 16 segment totals, lane l of every wave holding entries 4 l .. 4 l + 3
  // (ns * NW <= 256), their lane-inclusive prefix and the total R
  const u128* pb = part + (size_t)b * ns * NW;
  const int lane = threadIdx.x & 63;
  u128 pv[4], p4 = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    pv[u] = 4 * lane + u < ns * NW ? pb[4 * lane + u] : (u128)0;
    p4 += pv[u];
  }
  const u128 pinc = wave_incl_scan(p4);
  const u128 R = shfl_any(pinc, 63);
  int32_t tok;
  if (sp.greedy && pl.kind == 0) {
    tok = sp.argmax;
  } else if (pl.kind != 0 && R == 0) {
    // the residual is empty: draw from p itself (whole row, this workgroup)
    build_table(sp, c, tab_p);
    tok = draw_plain<false>(target + ((size_t)b * (k + 1) + pl.a) * V, sp, tab_p, pl.U, V, wt64, &found);
  } else {
    // target: floor(U Z / 2^24) for the bonus (Z = the kept mass of p), U R scaled for
    // a residual; then the slice whose running total passes it
    const u128 tgt = pl.kind == 0 ? (u128)(((u128)pl.U * sp.Z) >> 24) : scaled_target(pl.U, R);
    // the segment whose running total passes it: its lane walks its 4 entries
    int i_hit = -1;
    u128 before = pinc - p4;
    if (before <= tgt && pinc > tgt) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (i_hit < 0 && before + pv[u] > tgt) i_hit = 4 * lane + u;
        if (i_hit < 0) before += pv[u];
      }
    }
    const uint64_t owner = __ballot(i_hit >= 0);
    if (owner) {
      const int ol = __ffsll((unsigned long long)owner) - 1;
      i_hit = __shfl(i_hit, ol, 64);
      before = shfl_any(before, ol);
    } else {   // not reached for tgt < R
      i_hit = ns * NW - 1;
      before = R - pb[ns * NW - 1];
    }
    int lo, hi;
    split_range(nch, ns, i_hit / NW, lo, hi);
    const int seg = range_seg(lo, hi);
    const int lo1 = min(hi, lo + (i_hit % NW) * seg), hi1 = min(lo1 + seg, hi);
    with_draw(pl, target, draft, k, V, c, st_t, st_d, b, tab_p, tab_q, [&](auto ld, auto wt, auto tag) {
      using Acc = decltype(tag);
      Acc* wtot;
      if constexpr (sizeof(Acc) == 16) wtot = wt128; else wtot = wt64;
      draw_totals<Acc, 1>(lo1, hi1, ld, wt, wtot);
      tok = draw_find<Acc>(lo1, hi1, ld, wt, wtot, (Acc)(tgt - before), V, &found);
    });
  }
  if (threadIdx.x == 0) {
    n_accepted[b] = pl.a;
    next_token[b] = tok;
  }
}

__global__ __launch_bounds__(SP_THREADS) void sample_rows_kernel(
    const uint16_t* __restrict__ logits, int V, float inv_temp, uint64_t seed, uint64_t offset_arg,
    const uint64_t* __restrict__ offset_dev, int row_base, int slot,
    const RowStat* __restrict__ stats, int32_t* __restrict__ out) {
  __shared__ uint64_t wt64[SP_THREADS / 64];
  __shared__ int32_t found;
  __shared__ uint64_t tab[SP_NBINS];
  const int r = blockIdx.x;
  const uint64_t offset = offset_dev ? *offset_dev : offset_arg;
  const RowStat sp = stats[r];
  const float c = inv_temp * 1.44269504088896341f;
  const uint32_t U = philox_u24(seed, offset, (uint32_t)(row_base + r), (uint32_t)slot);
  build_table(sp, c, tab);
  __syncthreads();
  const int32_t tok = draw_plain<true>(logits + (size_t)r * V, sp, tab, U, V, wt64, &found);
  if (threadIdx.x == 0) out[r] = tok;
}

// Repetition penalty (src/generate.py:18-22) in place on bf16 logit rows: a token of the
// row's penalty set becomes bf16(x / p) if x > 0 else bf16(x * p), computed in fp32 as
// torch computes bf16 arithmetic (one rounding of the fp32 quotient / product to bf16).
// Grid (word blocks, rows): a thread owns one 32-bit word of the sequence's seen bitmap,
// i.e. 32 consecutive tokens, so no two threads touch the same token; thread 0 of
// block 0 of row (b, t) also applies the extra tokens (the drafts verified before
// position t), each once, skipping those already in the bitmap.
__device__ __forceinline__ void penalise(uint16_t* p, float pen) {
  const float x = __uint_as_float((uint32_t)*p << 16);
  const float y = x > 0.f ? x / pen : x * pen;
  *p = f32_to_bf16(y);
}

__global__ __launch_bounds__(256) void repetition_penalty_kernel(
    uint16_t* __restrict__ logits, long long ld, int T, int V, const uint32_t* __restrict__ seen,
    int words, const int32_t* __restrict__ extra, int extra_stride, int n0, float pen) {
  const int row = blockIdx.y, b = row / T, t = row - b * T;
  uint16_t* x = logits + (size_t)row * ld;
  const uint32_t* sb = seen + (size_t)b * words;
  const int w = blockIdx.x * 256 + threadIdx.x;
  const int wmax = (V + 31) / 32;
  if (w < wmax) {
    uint32_t bits = sb[w];
    while (bits) {
      const int bit = __ffs(bits) - 1;
      bits &= bits - 1;
      const int tok = 32 * w + bit;
      if (tok < V) penalise(x + tok, pen);
    }
  }
  if (extra && blockIdx.x == 0 && threadIdx.x == 0) {
    const int32_t* e = extra + (size_t)b * extra_stride;
    const int n = n0 + t;
    for (int j = 0; j < n; ++j) {
      const int tok = e[j];
      if (tok < 0 || tok >= V || ((sb[tok >> 5] >> (tok & 31)) & 1u)) continue;
      bool dup = false;
      for (int i = 0; i < j; ++i) dup |= e[i] == tok;
      if (!dup) penalise(x + tok, pen);
    }
  }
}

// seen[b] |= {tok[b * tok_stride + i] : i < n} (tokens outside [0, V) ignored).
__global__ void seen_mark_kernel(uint32_t* __restrict__ seen, int words,
                                 const int32_t* __restrict__ tok, long long tok_stride, int n,
                                 int V) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int t = tok[(size_t)b * tok_stride + i];
  if (t >= 0 && t < V) atomicOr(&seen[(size_t)b * words + (t >> 5)], 1u << (t & 31));
}

__global__ void philox_kernel(uint64_t seed, uint64_t offset, int rows, int slots, uint32_t* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows * slots) out[i] = philox_u24(seed, offset, (uint32_t)(i / slots), (uint32_t)(i % slots));
}

}  // namespace lollm

using namespace lollm;

static bool sampler_args_ok(int V, float top_p, float inv_temp) {
  if (V <= 0 || V % 8) return false;
  if (!(top_p == top_p)) return false;
  if (inv_temp > 0.0f && inv_temp < 1e-3f) return false;  // temperatures above 1000
  return true;
}

// Row statistics for rows0 rows of x0 followed by rows1 rows of x1 (one RowStat array):
// the histogram kernel for all of them in one launch, or for greedy rows the split
// argmax (partials at `part`).
static int launch_row_stats(const uint16_t* x0, int rows0, const uint16_t* x1, int rows1, int V,
                            float inv_temp, int top_k, float top_p, RowStat* st, uint64_t* part,
                            hipStream_t s) {
  if (inv_temp > 0.0f) {
    hipLaunchKernelGGL(row_stats_kernel, dim3(rows0 + rows1), dim3(SP_THREADS), 0, s, x0, rows0,
                       x1, V, inv_temp, top_k, top_p, st);
    return launch_status();
  }
  const uint16_t* xs[2] = {x0, x1};
  const int rs[2] = {rows0, rows1};
  int base = 0;
  for (int h = 0; h < 2; ++h) {
    if (rs[h] <= 0) continue;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(SP_NSPLIT, rs[h]), dim3(256), 0, s, xs[h], V,
                       part + (size_t)base * SP_NSPLIT);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rs[h]), dim3(64), 0, s,
                       (const uint64_t*)(part + (size_t)base * SP_NSPLIT), st + base,
                       (int32_t*)nullptr);
    if ((rc = launch_status())) return rc;
    base += rs[h];
  }
  return 0;
}

static long long stats_bytes(long long rows) {
  return rows * (long long)(sizeof(RowStat) + SP_NSPLIT * sizeof(uint64_t));
}

constexpr int SP_MAXSLICE = 16;   // vocabulary slices of the acceptance draw

static int accept_slices(int B) { return std::max(1, std::min(SP_MAXSLICE, 256 / B)); }

static long long accept_part_offset(int B, int k, int with_draft) {
  const long long st = stats_bytes((long long)B * (k + 1) + (with_draft ? (long long)B * k : 0));
  return (st + 15) / 16 * 16;
}

LOLLM_API long long lollm_spec_workspace_bytes(int B, int k, int with_draft) {
  if (B <= 0 || k < 0) return -1;
  // one u128 per (sequence, slice, wave)
  return accept_part_offset(B, k, with_draft) +
         (long long)B * accept_slices(B) * (SP_THREADS / 64) * (long long)sizeof(u128);
}

LOLLM_API long long lollm_sample_workspace_bytes(int rows) {
  if (rows <= 0) return -1;
  return stats_bytes(rows);
}

// lollm_spec_accept and lollm_spec_accept_rowmax: with target_rmax, the target rows'
// statistics take their maxima from those slots (one read per row); draft rows, and
// every row without target_rmax, the full row_stats pass.
static int spec_accept_impl(const void* target, const uint16_t* target_rmax, long long rmax_ld,
                            int rmax_slots, const void* draft, const int32_t* drafts, int B, int k,
                            int V, float inv_temperature, int top_k, float top_p, uint64_t seed,
                            uint64_t offset, const uint64_t* offset_dev, int32_t* n_accepted,
                            int32_t* next_token, void* workspace, long long workspace_bytes,
                            void* stream) {
  if (!target || !n_accepted || !next_token || !workspace || B <= 0 || k < 0) return LOLLM_EINVAL;
  if (k > 0 && !drafts) return LOLLM_EINVAL;
  if (k > 64) return LOLLM_EUNSUPPORTED;
  if (!sampler_args_ok(V, top_p, inv_temperature)) return LOLLM_EUNSUPPORTED;
  if (workspace_bytes < lollm_spec_workspace_bytes(B, k, draft != nullptr)) return LOLLM_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const int rt = B * (k + 1), rd = draft ? B * k : 0;
  RowStat* st_t = (RowStat*)workspace;
  RowStat* st_d = st_t + rt;
  uint64_t* part = (uint64_t*)(st_d + rd);
  int rc;
  if (target_rmax && inv_temperature > 0.0f) {
    hipLaunchKernelGGL(row_stats_known_kernel, dim3(rt), dim3(SP_THREADS), 0, st,
                       (const uint16_t*)target, V, inv_temperature, top_k, top_p, st_t, target_rmax,
                       rmax_ld, rmax_slots);
    if ((rc = launch_status())) return rc;
    rc = k > 0 && rd > 0 ? launch_row_stats((const uint16_t*)draft, rd, nullptr, 0, V,
                                            inv_temperature, top_k, top_p, st_d, part, st)
                         : 0;
  } else {
    rc = launch_row_stats((const uint16_t*)target, rt, (const uint16_t*)draft, k > 0 ? rd : 0, V,
                          inv_temperature, top_k, top_p, st_t, part, st);
  }
  if (rc) return rc;
  // the draw: B x ns workgroups sum the draw's weights over ns vocabulary slices (one
  // round of workgroups: one 1024-thread workgroup fits a CU), then one workgroup per
  // sequence finds the slice and the token in it
  const int ns = accept_slices(B);
  u128* apart = (u128*)((char*)workspace + accept_part_offset(B, k, draft != nullptr));
  const size_t tabs = (draft ? 2 : 1) * SP_NBINS * sizeof(uint64_t);
  static bool lds_set[64] = {};   // per device: the attribute is set on the current device
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return LOLLM_EUNSUPPORTED;
  if (!lds_set[dev]) {
    const int mx = 2 * SP_NBINS * (int)sizeof(uint64_t);
    hipError_t e = hipFuncSetAttribute((const void*)spec_partial_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, mx);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)spec_final_kernel,
                              hipFuncAttributeMaxDynamicSharedMemorySize, mx);
    if (e != hipSuccess) return LOLLM_EHIP_BASE + (int)e;
    lds_set[dev] = true;
  }
  hipLaunchKernelGGL(spec_partial_kernel, dim3(ns, B), dim3(SP_THREADS), tabs, st,
                     (const uint16_t*)target, (const uint16_t*)draft, drafts, k, V, inv_temperature,
                     seed, offset, offset_dev, st_t, draft ? st_d : nullptr, ns, apart);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(spec_final_kernel, dim3(B), dim3(SP_THREADS), tabs, st, (const uint16_t*)target,
                     (const uint16_t*)draft, drafts, k, V, inv_temperature, seed, offset, offset_dev,
                     st_t, draft ? st_d : nullptr, ns, (const u128*)apart, n_accepted, next_token);
  return launch_status();
}

LOLLM_API int lollm_spec_accept(const void* target, const void* draft, const int32_t* drafts,
                                int B, int k, int V, float inv_temperature, int top_k, float top_p,
                                uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                                int32_t* n_accepted, int32_t* next_token, void* workspace,
                                long long workspace_bytes, void* stream) {
  return spec_accept_impl(target, nullptr, 0, 0, draft, drafts, B, k, V, inv_temperature, top_k,
                          top_p, seed, offset, offset_dev, n_accepted, next_token, workspace,
                          workspace_bytes, stream);
}

LOLLM_API int lollm_spec_accept_rowmax(const void* target, const uint16_t* target_rowmax,
                                       long long rowmax_ld, int rowmax_slots, const void* draft,
                                       const int32_t* drafts, int B, int k, int V,
                                       float inv_temperature, int top_k, float top_p,
                                       uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                                       int32_t* n_accepted, int32_t* next_token, void* workspace,
                                       long long workspace_bytes, void* stream) {
  if (!target_rowmax || rowmax_slots <= 0 || rowmax_ld < rowmax_slots) return LOLLM_EINVAL;
  return spec_accept_impl(target, target_rowmax, rowmax_ld, rowmax_slots, draft, drafts, B, k, V,
                          inv_temperature, top_k, top_p, seed, offset, offset_dev, n_accepted,
                          next_token, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------- allocation-free
// lollm_spec_accept for callers that cannot allocate: its workspace (row statistics and
// draw partials, every byte written before it is read, so nothing needs clearing) lives
// in this fixed per-device array.  The host never uses the array's name as an address:
// each device's copy is located once with hipGetSymbolAddress, with that device current.
static __device__ __attribute__((aligned(256))) unsigned char scratch[LOLLM_SPEC_SCRATCH_BYTES];

static void* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return LOLLM_EHIP_BASE + (int)e;
  if (dev < 0 || dev >= 64) return LOLLM_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return LOLLM_EHIP_BASE + (int)e;
    if (!p) return LOLLM_EHIP_BASE + (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LOLLM_OK;
}

LOLLM_API int lollm_spec_accept_noalloc(const void* target, const void* draft,
                                        const int32_t* drafts, int B, int k, int V,
                                        float inv_temperature, int top_k, float top_p,
                                        uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                                        int32_t* n_accepted, int32_t* next_token, void* stream) {
  const long long need = lollm_spec_workspace_bytes(B, k, draft != nullptr);
  if (need < 0) return LOLLM_EINVAL;
  if (need > (long long)LOLLM_SPEC_SCRATCH_BYTES) return LOLLM_EUNSUPPORTED;
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return lollm_spec_accept(target, draft, drafts, B, k, V, inv_temperature, top_k, top_p, seed,
                           offset, offset_dev, n_accepted, next_token, ws,
                           (long long)LOLLM_SPEC_SCRATCH_BYTES, stream);
}

LOLLM_API int lollm_sample_rows(const void* logits, int rows, int V, float inv_temperature,
                                int top_k, float top_p, uint64_t seed, uint64_t offset,
                                const uint64_t* offset_dev, int row_base, int slot, int32_t* out,
                                void* workspace, long long workspace_bytes, void* stream) {
  if (!logits || !out || !workspace || rows <= 0 || slot < 0) return LOLLM_EINVAL;
  if (!sampler_args_ok(V, top_p, inv_temperature)) return LOLLM_EUNSUPPORTED;
  if (workspace_bytes < stats_bytes(rows)) return LOLLM_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  RowStat* stats = (RowStat*)workspace;
  uint64_t* part = (uint64_t*)(stats + rows);
  if (!(inv_temperature > 0.0f)) {  // greedy: the split argmax writes the tokens directly
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(SP_NSPLIT, rows), dim3(256), 0, st,
                       (const uint16_t*)logits, V, part);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, st, (const uint64_t*)part,
                       (RowStat*)nullptr, out);
    return launch_status();
  }
  int rc = launch_row_stats((const uint16_t*)logits, rows, nullptr, 0, V, inv_temperature, top_k,
                            top_p, stats, part, st);
  if (rc) return rc;
  hipLaunchKernelGGL(sample_rows_kernel, dim3(rows), dim3(SP_THREADS), 0, st,
                     (const uint16_t*)logits, V, inv_temperature, seed, offset, offset_dev, row_base,
                     slot, stats, out);
  return launch_status();
}

LOLLM_API int lollm_philox_uniform_u24(uint64_t seed, uint64_t offset, int rows, int slots,
                                       uint32_t* out, void* stream) {
  if (!out || rows <= 0 || slots <= 0) return LOLLM_EINVAL;
  const int n = rows * slots;
  hipLaunchKernelGGL(philox_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     seed, offset, rows, slots, out);
  return launch_status();
}

LOLLM_API int lollm_repetition_penalty(void* logits, long long ld, int B, int T, int V,
                                       const uint32_t* seen, int words, const int32_t* extra,
                                       int extra_stride, int n_extra0, float penalty,
                                       void* stream) {
  if (!logits || !seen || B <= 0 || T <= 0 || V <= 0 || ld < V || n_extra0 < 0) return LOLLM_EINVAL;
  if (words < (V + 31) / 32 || (long long)B * T > 65535) return LOLLM_EINVAL;
  if (extra && extra_stride < n_extra0 + T - 1) return LOLLM_EINVAL;
  if (!(penalty > 0.f) || !(penalty < 3.0e38f)) return LOLLM_EINVAL;
  const int wmax = (V + 31) / 32;
  hipLaunchKernelGGL(repetition_penalty_kernel, dim3((wmax + 255) / 256, B * T), dim3(256), 0,
                     (hipStream_t)stream, (uint16_t*)logits, ld, T, V, seen, words, extra,
                     extra_stride, n_extra0, penalty);
  return launch_status();
}

LOLLM_API int lollm_seen_mark(uint32_t* seen, int words, int B, const int32_t* tok,
                              long long tok_stride, int n, int V, void* stream) {
  if (!seen || !tok || B <= 0 || B > 65535 || n < 0 || V <= 0 || words < (V + 31) / 32 ||
      tok_stride < n)
    return LOLLM_EINVAL;
  if (n == 0) return LOLLM_OK;
  hipLaunchKernelGGL(seen_mark_kernel, dim3((n + 255) / 256, B), dim3(256), 0, (hipStream_t)stream,
                     seen, words, tok, tok_stride, n, V);
  return launch_status();
}

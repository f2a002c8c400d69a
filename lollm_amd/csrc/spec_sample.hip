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
//   row_stats    one 1024-thread workgroup per row, ONE pass over HBM: the row is
//                held in registers (19 x 16 B per thread covers V <= 155648; larger
//                rows re-read the tail), giving the max key (packed 16-bit order keys,
//                two tokens per max), then a per-key count histogram over the NBINS
//                keys below the max in LDS and block scans for the top-k / top-p cut
//                points and the kept mass Z;
//   argmax_*     greedy rows: the row split over 16 workgroups, partial maxima
//                merged by a second tiny kernel (a greedy row needs no histogram);
//   spec_partial / spec_final  the k accept tests in parallel, then the residual or
//                bonus draw in two passes: ns workgroups per sequence sum the draw's
//                weights over ns contiguous vocabulary slices, then one workgroup per
//                sequence locates the slice holding the target and the token in it;
//   sample_rows  one draw per row.
// A draw is an inverse CDF over token ids in two steps: every wave of the block
// sums the weights of its own contiguous sixteenth of the row (coalesced, one pass,
// exact integers), then the one wave whose segment holds the target walks it again
// with wave-level scans.  A token's weight depends only on its key's distance below
// the row maximum, so each draw first fills an LDS table of the NBINS weights (the
// same weight_of) and then reads one entry per token.  Residual masses are 64-bit
// when q is one-hot (argmax drafts) and 128-bit when q is a sampled distribution.
#include "common.h"

#include <algorithm>

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
// below the row's maximum key (zero past the cut) -- token_weight as a lookup.
__device__ void build_table(const RowStat& s, float c, uint64_t* tab) {
  const float xmax = key_value(s.kmax);
  for (int d = threadIdx.x; d < SP_NBINS; d += blockDim.x)
    tab[d] = (!s.greedy && d <= s.cut) ? weight_of(key_value(s.kmax - d), xmax, c) : 0;
}

__device__ __forceinline__ uint64_t table_weight(const RowStat& s, const uint64_t* tab,
                                                 uint32_t b, int32_t tok) {
  if (s.greedy) return tok == s.argmax ? 1u : 0u;
  const uint32_t d = (uint32_t)(s.kmax - skey(b));   // >= 0: kmax is the row maximum
  return d < (uint32_t)SP_NBINS ? tab[d] : 0;
}

// Order keys of the two bf16 in a word, packed (ord16 per half).
__device__ __forceinline__ uint32_t ord_pair(uint32_t w) {
  const uint32_t sgn = (w >> 15) & 0x00010001u;
  return w ^ ((sgn * 0x7FFFu) | 0x80008000u);
}

typedef unsigned short sp_us2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(sp_us2, a),
                                                                __builtin_bit_cast(sp_us2, b)));
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
constexpr int SP_REG = 19;       // 16-byte chunks per thread held in registers
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

__device__ __forceinline__ void hist_chunk(uint4 u, int32_t km, uint32_t* hist) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t b = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
    const int32_t d = km - skey(b);
    if (d < SP_NBINS) atomicAdd(&hist[d], 1u);
  }
}

// Sampled rows only (inv_temp > 0); greedy rows take the split argmax below.
__global__ __launch_bounds__(SP_THREADS) void row_stats_kernel(const uint16_t* __restrict__ logits,
                                                               int V, float inv_temp, int top_k,
                                                               float top_p, RowStat* stats) {
  __shared__ uint32_t hist[SP_NBINS];
  __shared__ uint64_t s64[16];
  __shared__ int32_t shared_cut;
  __shared__ uint64_t z_sh;
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int nch = V >> 3;
  const uint4* x4 = reinterpret_cast<const uint4*>(logits + (size_t)row * V);
  // ---- the row into registers (one HBM pass); zero the histogram meanwhile ----
  uint4 reg[SP_REG];
#pragma unroll
  for (int i = 0; i < SP_REG; ++i) {
    const int c = i * SP_THREADS + tid;
    reg[i] = c < nch ? x4[c] : make_uint4(0, 0, 0, 0);
  }
  for (int i = tid; i < SP_NBINS; i += SP_THREADS) hist[i] = 0;
  // ---- the maximum order key, two bf16 at a time ----
  uint32_t m2 = 0;
#pragma unroll
  for (int i = 0; i < SP_REG; ++i) {
    const int c = i * SP_THREADS + tid;
    if (c < nch) {
      m2 = max_u16x2(m2, ord_pair(reg[i].x));
      m2 = max_u16x2(m2, ord_pair(reg[i].y));
      m2 = max_u16x2(m2, ord_pair(reg[i].z));
      m2 = max_u16x2(m2, ord_pair(reg[i].w));
    }
  }
  for (int c = SP_REG * SP_THREADS + tid; c < nch; c += SP_THREADS) {
    const uint4 u = x4[c];
    m2 = max_u16x2(max_u16x2(m2, ord_pair(u.x)), max_u16x2(ord_pair(u.y), max_u16x2(ord_pair(u.z), ord_pair(u.w))));
  }
  const uint32_t omax = (uint32_t)block_max<uint64_t>((uint64_t)max((m2 & 0xFFFFu), (m2 >> 16)), s64);
  RowStat st;
  st.greedy = 0;
  st.argmax = -1;   // only greedy rows use it
  const int32_t km = skey(ord_bits(omax));   // skey is monotone in the order key
  st.kmax = km;
  // ---- per-key counts below the max (from registers) ----
#pragma unroll
  for (int i = 0; i < SP_REG; ++i) {
    const int c = i * SP_THREADS + tid;
    if (c < nch) hist_chunk(reg[i], km, hist);
  }
  for (int c = SP_REG * SP_THREADS + tid; c < nch; c += SP_THREADS) hist_chunk(x4[c], km, hist);
  __syncthreads();
  // ---- cut points and kept mass: thread t owns bins [8t, 8t + 8) ----
  constexpr int PER = SP_NBINS / SP_THREADS;
  const float xmax = key_value(km);
  const float c = inv_temp * 1.44269504088896341f;
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
  if (tid == 0) stats[row] = st;
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
// [lo, hi)), wt(raw, c, w[8]) turns it into the 8 token weights.  The totals pass keeps
// UN chunks per lane in flight.
__device__ __forceinline__ int range_seg(int lo, int hi) {
  return (hi - lo + SP_THREADS / 64 - 1) / (SP_THREADS / 64);
}

template <typename Acc, int UN, typename LD, typename WT>
__device__ Acc draw_totals(int lo, int hi, LD ld, WT wt, Acc* wtot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // wtot may still be read by a previous draw's waves
  const int seg = range_seg(lo, hi);
  const int c0 = lo + wave * seg, c1 = min(c0 + seg, hi);
  Acc acc = 0;
  for (int c = c0 + lane; c < c1; c += 64 * UN) {
    decltype(ld(0)) r[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) r[u] = ld(min(c + 64 * u, c1 - 1));
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      if (c + 64 * u < c1) {
        Acc w[8];
        wt(r[u], c + 64 * u, w);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += w[e];
      }
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

struct ChunkPair { u32x4_t p, q; };   // vector members: copies stay in registers

__device__ __forceinline__ u128 scaled_target(uint32_t U, u128 M) {
  return (u128)U * (M >> 24) + (((u128)U * (uint64_t)(M & 0xFFFFFFu)) >> 24);
}

// Plain draw from a row's own distribution p (u64 masses, target floor(U Z / 2^24));
// tab is p's weight table (build_table), complete before the call.
__device__ int32_t draw_plain(const uint16_t* xp, const RowStat& sp, const uint64_t* tab, uint32_t U,
                              int V, uint64_t* wtot, int32_t* found) {
  if (sp.greedy) return sp.argmax;
  const int nch = V >> 3;
  const u32x4_t* v4 = reinterpret_cast<const u32x4_t*>(xp);
  auto ld = [=](int ch) { return v4[ch]; };
  auto wt = [=](const u32x4_t& u, int ch, uint64_t* w) {
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      w[e] = table_weight(sp, tab, (wd[e >> 1] >> (16 * (e & 1))) & 0xFFFFu, ch * 8 + e);
  };
  draw_totals<uint64_t, 4>(0, nch, ld, wt, wtot);
  const uint64_t tgt = (uint64_t)(((u128)U * sp.Z) >> 24);
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
      const u32x4_t up = r.p, uq = r.q;
      const uint32_t pw[4] = {up.x, up.y, up.z, up.w}, qw[4] = {uq.x, uq.y, uq.z, uq.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = ch * 8 + e;
        const uint64_t wpt = table_weight(sp, tab_p, (pw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu, t);
        const uint64_t wqt = table_weight(sq, tab_q, (qw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu, t);
        const u128 l = (u128)wpt * Zq, r = (u128)wqt * sp.Z;
        w[e] = l > r ? l - r : (u128)0;
      }
    };
    f(ld, wt, (u128)0);
  } else if (pl.kind == 2) {
    // q one-hot at d: residual wp - [t == d] Zp fits 64 bits
    __syncthreads();
    const int d = pl.d;
    auto ld = [=](int ch) { return vp[ch]; };
    auto wt = [=](const u32x4_t& up, int ch, uint64_t* w) {
      const uint32_t pw[4] = {up.x, up.y, up.z, up.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = ch * 8 + e;
        const uint64_t wpt = table_weight(sp, tab_p, (pw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu, t);
        const uint64_t r = t == d ? sp.Z : 0;
        w[e] = wpt > r ? wpt - r : 0;
      }
    };
    f(ld, wt, (uint64_t)0);
  } else {
    // the bonus: p of row k itself
    __syncthreads();
    auto ld = [=](int ch) { return vp[ch]; };
    auto wt = [=](const u32x4_t& u, int ch, uint64_t* w) {
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        w[e] = table_weight(sp, tab_p, (wd[e >> 1] >> (16 * (e & 1))) & 0xFFFFu, ch * 8 + e);
    };
    f(ld, wt, (uint64_t)0);
  }
}

__device__ __forceinline__ void split_range(int nch, int ns, int s, int& lo, int& hi) {
  const int per = (nch + ns - 1) / ns;
  lo = min(nch, s * per);
  hi = min(nch, lo + per);
}

// Pass 1, grid (ns, B): workgroup (s, b) sums the draw's weights over the s-th of ns
// contiguous slices of the vocabulary (exact integers, u128 in part[b ns + s]).
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
    const Acc tot = draw_totals<Acc, sizeof(Acc) == 16 ? 2 : 4>(lo, hi, ld, wt, wtot);
    if (threadIdx.x == 0) part[(size_t)b * ns + s] = (u128)tot;
  });
}

// Pass 2, grid (B): the slice holding the target, then the token inside it.
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
  u128 R = 0;
  for (int s = 0; s < ns; ++s) R += part[(size_t)b * ns + s];
  int32_t tok;
  if (sp.greedy && pl.kind == 0) {
    tok = sp.argmax;
  } else if (pl.kind != 0 && R == 0) {
    // the residual is empty: draw from p itself (whole row, this workgroup)
    build_table(sp, c, tab_p);
    __syncthreads();
    tok = draw_plain(target + ((size_t)b * (k + 1) + pl.a) * V, sp, tab_p, pl.U, V, wt64, &found);
  } else {
    // target: floor(U Z / 2^24) for the bonus (Z = the kept mass of p), U R scaled for
    // a residual; then the slice whose running total passes it
    const u128 tgt = pl.kind == 0 ? (u128)(((u128)pl.U * sp.Z) >> 24) : scaled_target(pl.U, R);
    u128 before = 0;
    int s_hit = ns - 1;
    for (int s = 0; s < ns; ++s) {
      const u128 v = part[(size_t)b * ns + s];
      if (before + v > tgt) { s_hit = s; break; }
      before += v;
    }
    int lo, hi;
    split_range(nch, ns, s_hit, lo, hi);
    with_draw(pl, target, draft, k, V, c, st_t, st_d, b, tab_p, tab_q, [&](auto ld, auto wt, auto tag) {
      using Acc = decltype(tag);
      Acc* wtot;
      if constexpr (sizeof(Acc) == 16) wtot = wt128; else wtot = wt64;
      draw_totals<Acc, sizeof(Acc) == 16 ? 2 : 4>(lo, hi, ld, wt, wtot);
      tok = draw_find<Acc>(lo, hi, ld, wt, wtot, (Acc)(tgt - before), V, &found);
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
  const int32_t tok = draw_plain(logits + (size_t)r * V, sp, tab, U, V, wt64, &found);
  if (threadIdx.x == 0) out[r] = tok;
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

// Row statistics for `rows` rows: the histogram kernel, or for greedy rows the split
// argmax (partials at `part`).
static int launch_row_stats(const uint16_t* x, int rows, int V, float inv_temp, int top_k,
                            float top_p, RowStat* st, uint64_t* part, hipStream_t s) {
  if (inv_temp > 0.0f) {
    hipLaunchKernelGGL(row_stats_kernel, dim3(rows), dim3(SP_THREADS), 0, s, x, V, inv_temp,
                       top_k, top_p, st);
    return launch_status();
  }
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(SP_NSPLIT, rows), dim3(256), 0, s, x, V, part);
  int rc = launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, s, (const uint64_t*)part, st,
                     (int32_t*)nullptr);
  return launch_status();
}

static long long stats_bytes(long long rows) {
  return rows * (long long)(sizeof(RowStat) + SP_NSPLIT * sizeof(uint64_t));
}

constexpr int SP_MAXSLICE = 16;   // vocabulary slices of the acceptance draw

static long long accept_part_offset(int B, int k, int with_draft) {
  const long long st = stats_bytes((long long)B * (k + 1) + (with_draft ? (long long)B * k : 0));
  return (st + 15) / 16 * 16;
}

LOLLM_API long long lollm_spec_workspace_bytes(int B, int k, int with_draft) {
  if (B <= 0 || k < 0) return -1;
  return accept_part_offset(B, k, with_draft) + (long long)B * SP_MAXSLICE * (long long)sizeof(u128);
}

LOLLM_API long long lollm_sample_workspace_bytes(int rows) {
  if (rows <= 0) return -1;
  return stats_bytes(rows);
}

LOLLM_API int lollm_spec_accept(const void* target, const void* draft, const int32_t* drafts,
                                int B, int k, int V, float inv_temperature, int top_k, float top_p,
                                uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                                int32_t* n_accepted, int32_t* next_token, void* workspace,
                                long long workspace_bytes, void* stream) {
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
  int rc = launch_row_stats((const uint16_t*)target, rt, V, inv_temperature, top_k, top_p, st_t,
                            part, st);
  if (rc) return rc;
  if (draft && k > 0) {
    rc = launch_row_stats((const uint16_t*)draft, rd, V, inv_temperature, top_k, top_p, st_d,
                          part + (size_t)rt * SP_NSPLIT, st);
    if (rc) return rc;
  }
  // the draw: vocabulary slices summed by B x ns workgroups (about two per CU), then one
  // workgroup per sequence finds the slice and the token
  const int ns = std::max(1, std::min(SP_MAXSLICE, (512 + B - 1) / B));
  u128* apart = (u128*)((char*)workspace + accept_part_offset(B, k, draft != nullptr));
  // LDS: the weight table of p, and of q when the drafts are sampled (one-hot drafts
  // need only p's, which leaves room for two workgroups per CU)
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
  int rc = launch_row_stats((const uint16_t*)logits, rows, V, inv_temperature, top_k, top_p, stats,
                            part, st);
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

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
// Kernels: row_stats (one 1024-thread workgroup per row: max key / argmax, a
// per-key count histogram over the NBINS keys below the max held in LDS, then a
// block scan giving the top-k and top-p cut points and the kept mass Z);
// spec_accept (one workgroup per sequence: the k accept tests, then a block-scan
// inverse-CDF over one row for the residual or bonus draw); sample_rows.
#include "common.h"

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

__device__ __forceinline__ uint32_t bf16_at(const uint16_t* x, int i) { return x[i]; }

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

// ---------------------------------------------------------------- row statistics
__device__ void row_stats_block(const uint16_t* __restrict__ x, int V, float inv_temp, int top_k,
                                float top_p, RowStat* out, uint32_t* hist, uint64_t* s64,
                                int32_t* shared_cut) {
  const int tid = threadIdx.x;
  const int nch = V >> 3;
  const uint4* x4 = reinterpret_cast<const uint4*>(x);
  uint64_t best = 0;
  int32_t km = INT32_MIN;
  for (int c = tid; c < nch; c += SP_THREADS) {
    const uint4 u = x4[c];
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
  best = block_max<uint64_t>(best, s64);
  km = (int32_t)block_max<int64_t>((int64_t)km, reinterpret_cast<int64_t*>(s64));
  RowStat st;
  st.argmax = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
  st.kmax = km;
  st.greedy = !(inv_temp > 0.0f);
  if (st.greedy) {
    st.cut = 0;
    st.Z = 1;
    if (tid == 0) *out = st;
    return;
  }
  for (int i = tid; i < SP_NBINS; i += SP_THREADS) hist[i] = 0;
  __syncthreads();
  for (int c = tid; c < nch; c += SP_THREADS) {
    const uint4 u = x4[c];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t b = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      const int32_t d = km - skey(b);
      if (d < SP_NBINS) atomicAdd(&hist[d], 1u);
    }
  }
  __syncthreads();
  // thread t owns bins [8t, 8t + 8)
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
  if (tid == 0) *shared_cut = SP_NBINS - 1;
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
        if (run >= (uint64_t)top_k) { *shared_cut = tid * PER + j; break; }
      }
    }
    __syncthreads();
  }
  const int32_t cut_k = *shared_cut;
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
    __shared__ uint64_t z_sh;
    if (m0 <= tm && minc > tm) {
      uint64_t run = m0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        if (tid * PER + j > cut_k) break;
        run += mass[j];
        if (run > tm) { *shared_cut = tid * PER + j; z_sh = run; break; }
      }
    }
    __syncthreads();
    st.cut = *shared_cut;
    st.Z = z_sh;
  }
  if (tid == 0) *out = st;
}

__global__ __launch_bounds__(SP_THREADS) void row_stats_kernel(const uint16_t* __restrict__ logits,
                                                               int V, float inv_temp, int top_k,
                                                               float top_p, RowStat* stats) {
  __shared__ uint32_t hist[SP_NBINS];
  __shared__ uint64_t s64[16];
  __shared__ int32_t cut;
  const int row = blockIdx.x;
  row_stats_block(logits + (size_t)row * V, V, inv_temp, top_k, top_p, stats + row, hist, s64,
                  &cut);
}

// ---------------------------------------------------------------- inverse-CDF draw
// First token (in id order) whose inclusive prefix of wfn(token) exceeds `target`.
template <typename Acc, typename WFn>
__device__ int32_t block_draw(int V, Acc target, WFn wfn, Acc* scratch) {
  __shared__ int32_t found;
  const int tid = threadIdx.x;
  if (tid == 0) found = -1;
  __syncthreads();
  Acc run = 0;
  for (int base = 0; base < V; base += SP_THREADS * 8) {
    const int t0 = base + tid * 8;
    Acc w[8];
    Acc loc = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      w[e] = (t0 + e < V) ? wfn(t0 + e) : (Acc)0;
      loc += w[e];
    }
    Acc total;
    const Acc inc = block_inclusive_scan<Acc>(loc, scratch, &total);
    const Acc before = run + inc - loc;
    if (before <= target && run + inc > target) {
      Acc r = before;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        r += w[e];
        if (r > target) { found = t0 + e; break; }
      }
    }
    __syncthreads();
    if (found >= 0) break;
    run += total;
  }
  const int32_t f = found;
  __syncthreads();
  return f < 0 ? V - 1 : f;
}

__device__ __forceinline__ u128 scaled_target(uint32_t U, u128 M) {
  return (u128)U * (M >> 24) + (((u128)U * (uint64_t)(M & 0xFFFFFFu)) >> 24);
}

__global__ __launch_bounds__(SP_THREADS) void spec_accept_kernel(
    const uint16_t* __restrict__ target, const uint16_t* __restrict__ draft,
    const int32_t* __restrict__ drafts, int k, int V, float inv_temp, uint64_t seed,
    uint64_t offset_arg, const uint64_t* __restrict__ offset_dev, const RowStat* __restrict__ st_t,
    const RowStat* __restrict__ st_d, int32_t* __restrict__ n_accepted,
    int32_t* __restrict__ next_token) {
  __shared__ u128 scratch[16];
  __shared__ int32_t sh_a, sh_rej;
  const int b = blockIdx.x;
  const uint64_t offset = offset_dev ? *offset_dev : offset_arg;
  const float c = inv_temp * 1.44269504088896341f;
  if (threadIdx.x == 0) {
    int a = 0, rej = 0;
    for (int i = 0; i < k; ++i) {
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
      const uint32_t U = philox_u24(seed, offset, (uint32_t)b, (uint32_t)i);
      const u128 lhs = (u128)U * wq * Zp;
      const u128 rhs = ((u128)wp * Zq) << 24;
      if (!(lhs < rhs)) { rej = 1; break; }
      ++a;
    }
    sh_a = a;
    sh_rej = rej;
  }
  __syncthreads();
  const int a = sh_a;
  const uint32_t U = philox_u24(seed, offset, (uint32_t)b, (uint32_t)k);
  int32_t tok;
  if (!sh_rej) {
    const RowStat sp = st_t[b * (k + 1) + k];
    const uint16_t* xp = target + ((size_t)b * (k + 1) + k) * V;
    if (sp.greedy) {
      tok = sp.argmax;
    } else {
      const u128 tgt = ((u128)U * sp.Z) >> 24;
      tok = block_draw<u128>(V, tgt, [&](int t) { return (u128)token_weight(sp, c, xp[t], t); },
                             scratch);
    }
  } else {
    const RowStat sp = st_t[b * (k + 1) + a];
    const uint16_t* xp = target + ((size_t)b * (k + 1) + a) * V;
    int32_t d = drafts[b * k + a];
    d = d < 0 ? 0 : (d >= V ? V - 1 : d);
    RowStat sq;
    const uint16_t* xq = nullptr;
    uint64_t Zq = 1;
    if (draft) {
      sq = st_d[b * k + a];
      xq = draft + ((size_t)b * k + a) * V;
      Zq = sq.Z;
    }
    auto resid = [&](int t) -> u128 {
      const uint64_t wpt = token_weight(sp, c, xp[t], t);
      const uint64_t wqt = xq ? token_weight(sq, c, xq[t], t) : (uint64_t)(t == d);
      const u128 l = (u128)wpt * Zq, r = (u128)wqt * sp.Z;
      return l > r ? l - r : (u128)0;
    };
    // total residual mass
    u128 R = 0;
    for (int t = threadIdx.x; t < V; t += SP_THREADS) R += resid(t);
    R = block_sum<u128>(R, scratch);
    if (R == 0) {
      const u128 tgt = ((u128)U * sp.Z) >> 24;
      tok = sp.greedy ? sp.argmax
                      : block_draw<u128>(V, tgt, [&](int t) { return (u128)token_weight(sp, c, xp[t], t); },
                                         scratch);
    } else {
      tok = block_draw<u128>(V, scaled_target(U, R), resid, scratch);
    }
  }
  if (threadIdx.x == 0) {
    n_accepted[b] = a;
    next_token[b] = tok;
  }
}

__global__ __launch_bounds__(SP_THREADS) void sample_rows_kernel(
    const uint16_t* __restrict__ logits, int V, float inv_temp, uint64_t seed, uint64_t offset_arg,
    const uint64_t* __restrict__ offset_dev, int row_base, int slot,
    const RowStat* __restrict__ stats, int32_t* __restrict__ out) {
  __shared__ u128 scratch[16];
  const int r = blockIdx.x;
  const uint64_t offset = offset_dev ? *offset_dev : offset_arg;
  const RowStat sp = stats[r];
  const float c = inv_temp * 1.44269504088896341f;
  int32_t tok;
  if (sp.greedy) {
    tok = sp.argmax;
  } else {
    const uint16_t* xp = logits + (size_t)r * V;
    const uint32_t U = philox_u24(seed, offset, (uint32_t)(row_base + r), (uint32_t)slot);
    const u128 tgt = ((u128)U * sp.Z) >> 24;
    tok = block_draw<u128>(V, tgt, [&](int t) { return (u128)token_weight(sp, c, xp[t], t); },
                           scratch);
  }
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

LOLLM_API long long lollm_spec_workspace_bytes(int B, int k, int with_draft) {
  if (B <= 0 || k < 0) return -1;
  return (long long)(B * (k + 1) + (with_draft ? B * k : 0)) * (long long)sizeof(RowStat);
}

LOLLM_API int lollm_spec_accept(const void* target, const void* draft, const int32_t* drafts,
                                int B, int k, int V, float inv_temperature, int top_k, float top_p,
                                uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                                int32_t* n_accepted, int32_t* next_token, void* workspace,
                                long long workspace_bytes, void* stream) {
  if (!target || !n_accepted || !next_token || !workspace || B <= 0 || k < 0) return LOLLM_EINVAL;
  if (k > 0 && !drafts) return LOLLM_EINVAL;
  if (!sampler_args_ok(V, top_p, inv_temperature)) return LOLLM_EUNSUPPORTED;
  if (workspace_bytes < lollm_spec_workspace_bytes(B, k, draft != nullptr)) return LOLLM_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  RowStat* st_t = (RowStat*)workspace;
  RowStat* st_d = st_t + B * (k + 1);
  hipLaunchKernelGGL(row_stats_kernel, dim3(B * (k + 1)), dim3(SP_THREADS), 0, st,
                     (const uint16_t*)target, V, inv_temperature, top_k, top_p, st_t);
  int rc = launch_status();
  if (rc) return rc;
  if (draft && k > 0) {
    hipLaunchKernelGGL(row_stats_kernel, dim3(B * k), dim3(SP_THREADS), 0, st,
                       (const uint16_t*)draft, V, inv_temperature, top_k, top_p, st_d);
    if ((rc = launch_status())) return rc;
  }
  hipLaunchKernelGGL(spec_accept_kernel, dim3(B), dim3(SP_THREADS), 0, st, (const uint16_t*)target,
                     (const uint16_t*)draft, drafts, k, V, inv_temperature, seed, offset, offset_dev,
                     st_t, draft ? st_d : nullptr, n_accepted, next_token);
  return launch_status();
}

LOLLM_API int lollm_sample_rows(const void* logits, int rows, int V, float inv_temperature,
                                int top_k, float top_p, uint64_t seed, uint64_t offset,
                                const uint64_t* offset_dev, int row_base, int slot, int32_t* out,
                                void* workspace, long long workspace_bytes, void* stream) {
  if (!logits || !out || !workspace || rows <= 0 || slot < 0) return LOLLM_EINVAL;
  if (!sampler_args_ok(V, top_p, inv_temperature)) return LOLLM_EUNSUPPORTED;
  if (workspace_bytes < (long long)rows * (long long)sizeof(RowStat)) return LOLLM_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  RowStat* stats = (RowStat*)workspace;
  hipLaunchKernelGGL(row_stats_kernel, dim3(rows), dim3(SP_THREADS), 0, st,
                     (const uint16_t*)logits, V, inv_temperature, top_k, top_p, stats);
  int rc = launch_status();
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

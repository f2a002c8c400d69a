// Gated DeltaNet verify scan for gfx950.
//
// Math (src/qwen3_5/blocks.py:116-144), per (b, v-head h) and position t:
//   S <- S * exp(g_t);  d = (v_t - S^T k_t) * beta_t;  S <- S + k_t d^T;
//   o_t = S^T (q_t * q_scale)
// with optional L2 normalisation of q_t, k_t over Dk (blocks.py:54-56,124-125).
//
// Mapping: one 256-thread workgroup per (b, h); wave w owns the 32-column slab
// [32w, 32w + 32) of the 128 x 128 fp32 state, lane = (row group rg = lane / 8,
// column group cg = lane % 8) owns rows [16 rg, 16 rg + 16) x columns
// [32w + 4 cg, +4): 64 state floats in registers, loaded and stored as float4 so
// every wave instruction moves 8 full 128-byte rows.  Columns of the state are
// independent in the recurrence, so slabs never communicate; the reductions over
// Dk (S^T k, S^T q, k.q, |k|^2, |q|^2) are xor-shuffles across the 8 row groups.
// The decay is folded algebraically so each position is ONE pass over the state:
//   a = exp(g) S^T k,  d = (v - a) beta,  o = exp(g) S^T q + d (k.q),
//   S' = exp(g) S + k d^T   (and S'^T k_{t+1}, S'^T q_{t+1} accumulate in the same pass).
// State traffic per (b, h): read Dk*Dv*4 bytes once, write Dk*Dv*4 per snapshot.
#include "common.h"

namespace lollm {

constexpr int GDN_DK = 128;
constexpr int GDN_DV = 128;
constexpr int GDN_ROWS = 16;  // rows per lane

template <typename T>
__device__ __forceinline__ void load_rows(const T* p, float (&x)[GDN_ROWS]) {
#pragma unroll
  for (int r = 0; r < GDN_ROWS; ++r) x[r] = Elt<T>::load(p + r);
}

template <>
__device__ __forceinline__ void load_rows<uint16_t>(const uint16_t* p, float (&x)[GDN_ROWS]) {
  const uint4* p4 = reinterpret_cast<const uint4*>(p);
  uint4 a = p4[0], b = p4[1];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load_rows<float>(const float* p, float (&x)[GDN_ROWS]) {
  const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float4 f = p4[i];
    x[4 * i] = f.x; x[4 * i + 1] = f.y; x[4 * i + 2] = f.z; x[4 * i + 3] = f.w;
  }
}

// NC consecutive value / output columns of one row (4 per lane in the verify scan)
template <typename T, int NC>
__device__ __forceinline__ void load_cols(const T* p, float (&x)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) x[c] = Elt<T>::load(p + c);
}

template <typename T, int NC>
__device__ __forceinline__ void store_cols(T* p, const float (&x)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) Elt<T>::store(p + c, x[c]);
}

template <>
__device__ __forceinline__ void store_cols<uint16_t, 4>(uint16_t* p, const float (&x)[4]) {
  uint2 w;
  w.x = (uint32_t)f32_to_bf16(x[0]) | ((uint32_t)f32_to_bf16(x[1]) << 16);
  w.y = (uint32_t)f32_to_bf16(x[2]) | ((uint32_t)f32_to_bf16(x[3]) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}

// One lane's 4 state floats of a row: plain loads (the state is read once), streaming
// stores (a snapshot is read back at most once, by a later launch; sending it straight
// to HBM spares the end-of-launch write-back of dirty L2 lines)
__device__ __forceinline__ void load_state(const float* p, float (&x)[4]) {
  const float4 f = *reinterpret_cast<const float4*>(p);
  x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
}

__device__ __forceinline__ void store_state(float* p, const float (&x)[4]) {
  const u32x4_t w = {__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                     __float_as_uint(x[3])};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

template <typename T, bool L2>
__global__ __launch_bounds__(256) void gdn_verify_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ g, const T* __restrict__ beta, const float* state,
    const int32_t* __restrict__ state_slot, int state_slots, T* __restrict__ out,
    float* __restrict__ snapshots, float* final_state, int T_len, int Hk, int Hv,
    float q_scale) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int cg = lane & 7, rg = lane >> 3;
  const int bh = blockIdx.x;
  const int b = bh / Hv, h = bh - b * Hv;
  const int hk = h / (Hv / Hk);
  const int row0 = rg * GDN_ROWS;
  const int col0 = wave * 32 + cg * 4;
  constexpr int NC = 4;  // state columns per lane
  constexpr size_t SS = (size_t)GDN_DK * GDN_DV;

  float S[GDN_ROWS][NC];
  if (state != nullptr) {
    int slot = state_slot ? state_slot[b] : 0;
    slot = slot < 0 ? 0 : (slot >= state_slots ? state_slots - 1 : slot);  // never out of range
    const float* s0 = state + ((size_t)(b * state_slots + slot) * Hv + h) * SS;
#pragma unroll
    for (int r = 0; r < GDN_ROWS; ++r) load_state(s0 + (size_t)(row0 + r) * GDN_DV + col0, S[r]);
  } else {
#pragma unroll
    for (int r = 0; r < GDN_ROWS; ++r)
#pragma unroll
      for (int c = 0; c < NC; ++c) S[r][c] = 0.f;
  }

  // inputs of position t
  auto qk_ptr = [&](const T* base, int t) {
    return base + (((size_t)b * T_len + t) * Hk + hk) * GDN_DK + row0;
  };
  auto gi_of = [&](int t) { return ((size_t)b * T_len + t) * Hv + h; };
  float kr[GDN_ROWS], qr[GDN_ROWS];
  load_rows<T>(qk_ptr(k, 0), kr);
  load_rows<T>(qk_ptr(q, 0), qr);
  // g, beta and this lane's value columns are loaded one position ahead with k and q,
  // so no wait for them covers the previous position's snapshot stores (the memory
  // counter retires in issue order, stores included)
  float graw = g[gi_of(0)], braw = Elt<T>::load(beta + gi_of(0)), vv[NC];
  load_cols<T, NC>(v + gi_of(0) * GDN_DV + col0, vv);

  // partial dot products of the current state with k_t, q_t (this lane's rows)
  float pa[NC], pb[NC], pkq = 0.f, pkk = 0.f, pqq = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) pa[c] = pb[c] = 0.f;
#pragma unroll
  for (int r = 0; r < GDN_ROWS; ++r) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      pa[c] = fmaf(S[r][c], kr[r], pa[c]);
      pb[c] = fmaf(S[r][c], qr[r], pb[c]);
    }
    pkq = fmaf(kr[r], qr[r], pkq);
    if (L2) {
      pkk = fmaf(kr[r], kr[r], pkk);
      pqq = fmaf(qr[r], qr[r], pqq);
    }
  }

  for (int t = 0; t < T_len; ++t) {
    // prefetch the next position's k, q, g, beta, v while this one is reduced
    float kn[GDN_ROWS], qn[GDN_ROWS], gn = 0.f, bn = 0.f, vn[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) vn[c] = 0.f;
    const bool has_next = t + 1 < T_len;
    if (has_next) {
      load_rows<T>(qk_ptr(k, t + 1), kn);
      load_rows<T>(qk_ptr(q, t + 1), qn);
      gn = g[gi_of(t + 1)];
      bn = Elt<T>::load(beta + gi_of(t + 1));
      load_cols<T, NC>(v + gi_of(t + 1) * GDN_DV + col0, vn);
    }
    const size_t gi = gi_of(t);
    const float gam = __expf(graw);
    const float bet = braw;

    // reduce over the 8 row groups (lanes differing in bits 3..5)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      pa[c] = sum_lanes8(pa[c]);
      pb[c] = sum_lanes8(pb[c]);
    }
    pkq = sum_lanes8(pkq);
    if (L2) {
      pkk = sum_lanes8(pkk);
      pqq = sum_lanes8(pqq);
    }
    const float rk = L2 ? rsqrtf(pkk + 1e-6f) : 1.f;
    const float rq = (L2 ? rsqrtf(pqq + 1e-6f) : 1.f) * q_scale;
    const float kq = pkq * rk * rq;
    float d[NC], o[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      d[c] = (vv[c] - gam * pa[c] * rk) * bet;
      o[c] = gam * pb[c] * rq + d[c] * kq;
    }
    if (rg == 0) store_cols<T, NC>(out + gi * GDN_DV + col0, o);

    // one pass: decay + rank-1 update, snapshot, next position's partial dots
    float* snap = snapshots ? snapshots + (((size_t)b * T_len + t) * Hv + h) * SS : nullptr;
#pragma unroll
    for (int c = 0; c < NC; ++c) pa[c] = pb[c] = 0.f;
    pkq = pkk = pqq = 0.f;
#pragma unroll
    for (int r = 0; r < GDN_ROWS; ++r) {
      const float kk_r = kr[r] * rk;
#pragma unroll
      for (int c = 0; c < NC; ++c) S[r][c] = fmaf(kk_r, d[c], gam * S[r][c]);
      if (snap) store_state(snap + (size_t)(row0 + r) * GDN_DV + col0, S[r]);
      if (has_next) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          pa[c] = fmaf(S[r][c], kn[r], pa[c]);
          pb[c] = fmaf(S[r][c], qn[r], pb[c]);
        }
        pkq = fmaf(kn[r], qn[r], pkq);
        if (L2) {
          pkk = fmaf(kn[r], kn[r], pkk);
          pqq = fmaf(qn[r], qn[r], pqq);
        }
      }
    }
    if (has_next) {
#pragma unroll
      for (int r = 0; r < GDN_ROWS; ++r) { kr[r] = kn[r]; qr[r] = qn[r]; }
#pragma unroll
      for (int c = 0; c < NC; ++c) vv[c] = vn[c];
      graw = gn;
      braw = bn;
    }
  }

  if (final_state) {
    float* sf = final_state + ((size_t)b * Hv + h) * SS;
#pragma unroll
    for (int r = 0; r < GDN_ROWS; ++r) store_state(sf + (size_t)(row0 + r) * GDN_DV + col0, S[r]);
  }
}

// state_out[b, h] = snapshots[b, slot[b], h]: one float4 per thread.
__global__ __launch_bounds__(256) void gdn_select_kernel(const float4* __restrict__ snaps,
                                                         const int32_t* __restrict__ slot,
                                                         float4* __restrict__ out, int T_len,
                                                         int per_seq4) {
  const int b = blockIdx.y;
  int s = slot[b];
  s = s < 0 ? 0 : (s >= T_len ? T_len - 1 : s);  // never out of range
  const float4* src = snaps + ((size_t)b * T_len + s) * per_seq4;
  float4* dst = out + (size_t)b * per_seq4;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < per_seq4; i += gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace lollm

using namespace lollm;

LOLLM_API int lollm_gdn_verify(const void* q, const void* k, const void* v, const float* g,
                               const void* beta, const float* state, const int32_t* state_slot,
                               int state_slots, void* out, float* snapshots, float* final_state,
                               int B, int T, int Hk, int Hv, int Dk, int Dv, int dtype,
                               int qk_l2norm, float q_scale, void* stream) {
  if (!q || !k || !v || !g || !beta || !out) return LOLLM_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0 || Hv % Hk != 0) return LOLLM_EINVAL;
  if (state_slots < 1) return LOLLM_EINVAL;
  if (Dk != GDN_DK || Dv != GDN_DV) return LOLLM_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(B * Hv), block(256);
#define GDN_LAUNCH(TT, L2)                                                                  \
  hipLaunchKernelGGL((gdn_verify_kernel<TT, L2>), grid, block, 0, st, (const TT*)q,        \
                     (const TT*)k, (const TT*)v, g, (const TT*)beta, state, state_slot,     \
                     state_slots, (TT*)out, snapshots, final_state, T, Hk, Hv, q_scale)
  if (dtype == LOLLM_BF16) {
    if (qk_l2norm) GDN_LAUNCH(uint16_t, true); else GDN_LAUNCH(uint16_t, false);
  } else if (dtype == LOLLM_F32) {
    if (qk_l2norm) GDN_LAUNCH(float, true); else GDN_LAUNCH(float, false);
  } else {
    return LOLLM_EUNSUPPORTED;
  }
#undef GDN_LAUNCH
  return launch_status();
}

LOLLM_API int lollm_gdn_select_state(const float* snapshots, const int32_t* slot,
                                     float* state_out, int B, int T, int Hv, int Dk, int Dv,
                                     void* stream) {
  if (!snapshots || !slot || !state_out || B <= 0 || T <= 0 || Hv <= 0) return LOLLM_EINVAL;
  if (((size_t)Hv * Dk * Dv) % 4 != 0) return LOLLM_EUNSUPPORTED;
  const int per_seq4 = (int)((size_t)Hv * Dk * Dv / 4);
  dim3 grid((per_seq4 + 255) / 256 < 1024 ? (per_seq4 + 255) / 256 : 1024, B);
  hipLaunchKernelGGL(gdn_select_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const float4*)snapshots, slot, (float4*)state_out, T, per_seq4);
  return launch_status();
}

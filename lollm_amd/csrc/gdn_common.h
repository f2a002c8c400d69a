// Shared by the GDN layer kernels: the argument block, channel constants and the
// elementwise helpers (src/qwen3_5/blocks.py:268-329).
#pragma once

#include "common.h"

namespace lollm {

constexpr int GL_DK = 128;
constexpr int GL_TC = 8;         // tokens per chunk
constexpr int GL_KMAX = 4;       // conv kernel width (linear_conv_kernel_dim)
constexpr int GL_CH = 3 * GL_DK; // q, k, v channels per head

// Replay record of one position.  A short call (T <= S) does not store the state after
// each position; it stores what the delta rule consumed there, and the next call rebuilds
// the state after any accepted prefix from the committed state and these records:
//   bytes [0, 2 Dk)            k after conv + SiLU, bf16 (the scan reads bf16-rounded values)
//   bytes [2 Dk, 2 Dk + 2 Dv)  v, bf16
//   then fp32 gamma = exp(g), beta, 1 / sqrt(|k|^2 + 1e-6) and a zero pad word
constexpr int GL_REC_BYTES = 4 * GL_DK + 16;
constexpr int GL_REC_U4 = GL_REC_BYTES / 16;

struct GdnLayerArgs {
  const uint16_t* proj;      // (B, T, P): [qkv (C) | z (value_dim) | b (Hv) | a (Hv)]
  const uint16_t* conv_w;    // (C, K)
  const float* A_log;        // (Hv)
  const float* dt_bias;      // (Hv)
  const uint16_t* norm_w;    // (Dv)
  uint16_t* win;             // (B, 2 W, C) conv windows
  const int32_t* conv_off;   // (B) first committed-state row in win
  float* rec;                // (B, 2, Hv, Dk, Dv) recurrent state, two halves
  const int32_t* rec_half;   // (B) half of rec / rep holding the committed state
  uint8_t* rep;              // (B, 2, Hv, S, GL_REC_BYTES) replay records, halves as rec
  const int32_t* replay;     // (B) leading records of the committed half not in its state
  uint16_t* out;             // (B, T, value_dim)
  long long P;
  int T, Hk, Hv, C, key_dim, value_dim, K;
  int W, S, fresh;
  float eps;
};

// One thread's slice of a head's 128 x 128 fp32 state: rows row0 .. row0 + 15 (k index) x
// columns col0 .. col0 + 3 (v index); a wave holds 32 columns, lanes 8 apart hold the same
// columns.  pa = (S^T k) at the thread's columns after the xor reduction over row groups.
// The delta rule's update from pa, written once so that the scan and the replay of a
// record round identically:
//   d = (v - gamma pa / |k|) beta,   S = gamma S + (k / |k|) d^T
__device__ __forceinline__ void gdn_delta(float (&d)[4], const float (&pa)[4], const float (&vv)[4],
                                          float gam, float rk, float bet) {
#pragma unroll
  for (int c = 0; c < 4; ++c) d[c] = (vv[c] - gam * pa[c] * rk) * bet;
}
__device__ __forceinline__ void gdn_update(float (&S)[16][4], const float (&kr)[16], float rk,
                                           const float (&d)[4], float gam) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float k_r = kr[r] * rk;
#pragma unroll
    for (int c = 0; c < 4; ++c) S[r][c] = fmaf(k_r, d[c], gam * S[r][c]);
  }
}
// Apply one replay record (global or LDS address) to the thread's slice.
__device__ __forceinline__ void gdn_replay_one(float (&S)[16][4], const uint8_t* rp, int row0, int col0) {
  const uint4 k0 = *reinterpret_cast<const uint4*>(rp + 2 * row0);
  const uint4 k1 = *reinterpret_cast<const uint4*>(rp + 2 * row0 + 16);
  const uint2 v2 = *reinterpret_cast<const uint2*>(rp + 2 * GL_DK + 2 * col0);
  const float4 sc = *reinterpret_cast<const float4*>(rp + 4 * GL_DK);
  const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
  float kr[16], vv[4];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    kr[2 * e] = __uint_as_float(kw[e] << 16);
    kr[2 * e + 1] = __uint_as_float(kw[e] & 0xffff0000u);
  }
  vv[0] = __uint_as_float(v2.x << 16); vv[1] = __uint_as_float(v2.x & 0xffff0000u);
  vv[2] = __uint_as_float(v2.y << 16); vv[3] = __uint_as_float(v2.y & 0xffff0000u);
  float pa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) pa[c] = fmaf(S[r][c], kr[r], pa[c]);
#pragma unroll
  for (int c = 0; c < 4; ++c) pa[c] = sum_lanes8(pa[c]);
  float d[4];
  gdn_delta(d, pa, vv, sc.x, sc.z, sc.y);
  gdn_update(S, kr, sc.z, d, sc.x);
}
// The k | v part of position t's record from the conv output rows in LDS (bf16-exact
// fp32 values, so the truncation is exact): 32 chunks of 8 values, chunk `part`.
__device__ __forceinline__ uint4 gdn_record_kv(const float* act_row_k, int part) {
  const float* p = act_row_k + part * 8;
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w[e] = (__float_as_uint(p[2 * e]) >> 16) | (__float_as_uint(p[2 * e + 1]) & 0xffff0000u);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Host side, before a long call (T > S): launches the kernel that writes the committed
// state (the committed half's state + its replay records) into the other half, where the
// long-call kernels start from (defined in gdn_layer.hip).
int gdn_long_call_prologue(const GdnLayerArgs& a, int B, hipStream_t stream);

// SiLU with the hardware reciprocal: within 1.5 ulp (fp32) of x / (1 + e^-x), below the
// resolution of the bf16 values it feeds
__device__ __forceinline__ float silu_g(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

__device__ __forceinline__ float softplus_g(float x) {  // torch: linear above 20
  return x > 20.f ? x : log1pf(__expf(x));
}

// Workgroup barrier that orders LDS only: outstanding global loads and stores (the
// snapshot stream) are not waited for.
__device__ __forceinline__ void lds_only_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace lollm

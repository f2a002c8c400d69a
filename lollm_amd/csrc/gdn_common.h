// Shared by the GDN layer kernels: the argument block, channel constants and the
// elementwise helpers (src/qwen3_5/blocks.py:268-329).
#pragma once

#include "common.h"

namespace lollm {

constexpr int GL_DK = 128;
constexpr int GL_TC = 8;         // tokens per chunk
constexpr int GL_KMAX = 4;       // conv kernel width (linear_conv_kernel_dim)
constexpr int GL_CH = 3 * GL_DK; // q, k, v channels per head

struct GdnLayerArgs {
  const uint16_t* proj;      // (B, T, P): [qkv (C) | z (value_dim) | b (Hv) | a (Hv)]
  const uint16_t* conv_w;    // (C, K)
  const float* A_log;        // (Hv)
  const float* dt_bias;      // (Hv)
  const uint16_t* norm_w;    // (Dv)
  uint16_t* win;             // (B, 2 W, C) conv windows
  const int32_t* conv_off;   // (B) first committed-state row in win
  float* rec;                // (B, 2 S, Hv, Dk, Dv) recurrent-state snapshots
  const int32_t* rec_slot;   // (B) committed-state slot in rec
  uint16_t* out;             // (B, T, value_dim)
  long long P;
  int T, Hk, Hv, C, key_dim, value_dim, K;
  int W, S, fresh;
  float eps;
};

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

// Shared helpers for the lollm_amd HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lollm_amd.h"

#define LOLLM_API extern "C" __attribute__((visibility("default")))

namespace lollm {

// ---- bf16 <-> fp32 (round to nearest even, like torch) ----
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Element loads/stores for the two activation dtypes the kernels accept.
template <typename T> struct Elt;
template <> struct Elt<float> {
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float v) { *p = v; }
};
template <> struct Elt<uint16_t> {
  __device__ static float load(const uint16_t* p) { return bf16_to_f32(*p); }
  __device__ static void store(uint16_t* p, float v) { *p = f32_to_bf16(v); }
};

__device__ __forceinline__ float wave_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Streaming (non-temporal) 16-byte global load/store: data touched once per launch
// should not displace reusable lines in L2 / MALL.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(void* p, uint4 v) {
  u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LOLLM_OK : LOLLM_EHIP_BASE + (int)e;
}

}  // namespace lollm

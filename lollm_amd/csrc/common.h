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

// Sum over the 8 lanes of a wave that share lane % 8 (partners 8, 16 and 32 lanes away),
// the same value in each of them: a DPP rotation by 8 inside each 16-lane row, then the
// gfx950 row swaps (v_permlane16_swap, v_permlane32_swap) for the partners in the other
// row of the pair and in the other half.  Every step adds a lane's value and its
// partner's, so the sums and their rounding are those of the xor-shuffle tree
// (v + shfl_xor(v, 8), then 16, then 32) without its LDS-crossbar round trips.
__device__ __forceinline__ float sum_lanes8(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128 /* row_ror:8 */,
                                                  0xf, 0xf, false));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sum over each 16-lane row of a wave (lanes 16 r .. 16 r + 15), the same value in each
// lane, with DPP only: partners 1 and 2 away (quad permutes), 4 away (after the first two
// steps every lane of a quad holds the quad's sum, and the half-row mirror reads the other
// quad) and 8 away (row rotation).  The sums are those of the xor-shuffle tree over masks
// 1, 2, 4, 8.
__device__ __forceinline__ float sum_lanes16(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1 /* quad 1,0,3,2 */, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e /* quad 2,3,0,1 */, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141 /* row_half_mirror */, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128 /* row_ror:8 */, 0xf, 0xf, false));
  return v;
}

// Streaming (non-temporal) 16-byte global load/store: data touched once per launch
// should not displace reusable lines in L2 / MALL.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
// Buffer descriptor over [base, base + bytes): loads at offsets past the end return zero
// and touch no memory (bytes = 0 gives a descriptor whose loads are all zero).  Base and
// size are made explicitly uniform (scalar registers).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  const uint64_t pu = ((uint64_t)hi << 32) | (uint64_t)lo;   // no sign extension of the low word
  return __builtin_amdgcn_make_buffer_rsrc((void*)pu, (short)0,
                                           __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000);
}
__device__ __forceinline__ void store_nt(void* p, uint4 v) {
  u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

// Sum over a workgroup of THREADS threads (wave64); red holds THREADS / 64 floats.
template <int THREADS>
__device__ __forceinline__ float block_sum_f(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) t += red[w];
  return t;
}

// RMSNorm arithmetic shared by every kernel that normalises a hidden row, so fused and
// stand-alone paths give the same bits: a RMS_THREADS-thread workgroup per row, thread t
// owns the 8-value chunks t and t + RMS_THREADS (rows of up to 8192), accumulates the
// squares in chunk order, then rstd = rsqrt(block sum / H + eps) and
// y = bf16(v * rstd * (1 + w)).
constexpr int RMS_THREADS = 512;
constexpr int RMS_CHUNKS = 2;
__device__ __forceinline__ float rms_rstd(float ss, float* red, int H, float eps) {
  return rsqrtf(block_sum_f<RMS_THREADS>(ss, red) / (float)H + eps);
}
__device__ __forceinline__ uint32_t rms_out2(float v0, float v1, float r, uint32_t w2) {
  const float w0 = __uint_as_float(w2 << 16), w1 = __uint_as_float(w2 & 0xffff0000u);
  return f32_to_bf16(v0 * r * (1.f + w0)) | ((uint32_t)f32_to_bf16(v1 * r * (1.f + w1)) << 16);
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LOLLM_OK : LOLLM_EHIP_BASE + (int)e;
}

}  // namespace lollm

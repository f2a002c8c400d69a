// Gated GQA attention over a per-sequence KV cache for the 1 + k verify block
// (gfx950, bf16 MFMA 32x32x16).
//
// Math (src/qwen3_5/blocks.py:226-235 + src/attention.py:43-51): query i of the T
// new positions of sequence b sits at absolute position L_b - T + i and attends the
// keys at positions <= that (offset-causal; plain causal when T == L_b); scores are
// scaled by D^-0.5; q-head h reads KV head h / n_rep (blocks.py:152-156, no
// expansion is materialised); the output is o * sigmoid(gate) (blocks.py:235).
//
// Mapping: a workgroup (4 waves) = (split of `chunk` keys, KV head x query block,
// sequence).  The 32 MFMA rows pack n_rep q-heads x QB queries of one KV head, so
// every K/V byte streamed from HBM serves all the q-heads that share it.  The split
// is walked in 64-key blocks:
//   - the workgroup stages the K and V block in LDS with coalesced 16-byte loads
//     (the next block's loads are in flight while this one is computed; barriers
//     only wait for LDS, never for those loads);
//   - wave w computes S^T for keys [16w, 16w+16) x 32 rows (16x16x32 MFMA, K from
//     LDS, Q^T held in registers); masked row maxima are exchanged through LDS and
//     every wave applies the same running max; P^T goes to LDS as bf16;
//   - wave w owns head-dim columns [64w, 64w+64) of O^T (32x32x16 MFMA, A = V^T read
//     from LDS, B = P^T), so O needs only 32 accumulators per wave and no merge.
// A split writes (m, l, O) partials; a combine kernel merges the splits and applies
// the gate (a single-split sequence finishes in place).
#include "common.h"

namespace lollm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AT_D = 256;            // head dim
constexpr int AT_ROWS = 32;          // MFMA rows per workgroup (n_rep x QB)
constexpr int AT_BLOCK = 64;         // keys per workgroup iteration
constexpr int AT_WAVES = 4;
constexpr int AT_KROW = AT_D * 2 + 16;        // padded bytes per K / V row in LDS
constexpr int AT_PROW = AT_BLOCK * 2 + 16;    // padded bytes per P^T row in LDS
constexpr int AT_OROW = AT_D + 1;             // padded floats per O row in LDS
constexpr int AT_PART = 2 * AT_ROWS + AT_ROWS * AT_D;  // floats per split partial
constexpr int AT_LDS_K = 0;
constexpr int AT_LDS_V = AT_LDS_K + AT_BLOCK * AT_KROW;
constexpr int AT_LDS_P = AT_LDS_V + AT_BLOCK * AT_KROW;
constexpr int AT_LDS_M = AT_LDS_P + AT_ROWS * AT_PROW;
constexpr int AT_LDS_BYTES = AT_LDS_M + 2 * AT_WAVES * AT_ROWS * 4;

struct AttnArgs {
  const uint16_t* q;       // (B, T, Hq, D)
  const uint16_t* kc;      // K cache
  const uint16_t* vc;      // V cache
  const int32_t* kv_len;   // (B) keys per sequence, the T new ones included
  const uint16_t* gate;    // (B, T, Hq * D) or null
  uint16_t* out;           // (B, T, Hq * D)
  float* ws;               // partials
  long long seq_stride, head_stride;  // cache strides in elements
  int T, Hq, Hkv, n_rep, QB, qblocks, chunk, max_splits, max_len;
  float cl2;               // scale * log2(e)
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

// Workgroup barrier that orders LDS only: global loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ __launch_bounds__(256, 2) void attn_verify_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int split = blockIdx.x;
  const int kvh = blockIdx.y / a.qblocks, qb = blockIdx.y % a.qblocks;
  const int b = blockIdx.z;
  const int L = min(max(a.kv_len[b], 0), a.max_len);  // never past the cache capacity
  const int nsplit = (L + a.chunk - 1) / a.chunk;
  if (split >= nsplit) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4, l32 = lane & 31, h2 = lane >> 5;
  const int q0 = qb * a.QB;
  const int QB = min(a.QB, a.T - q0);
  const int rows = a.n_rep * QB;

  unsigned char* k_lds = smem + AT_LDS_K;
  unsigned char* v_lds = smem + AT_LDS_V;
  unsigned char* p_lds = smem + AT_LDS_P;
  float* m_lds = reinterpret_cast<float*>(smem + AT_LDS_M);    // [wave][row]
  float* l_lds = m_lds + AT_WAVES * AT_ROWS;

  // ---- Q (rows r = hr * QB + i) staged through LDS into B operands ----
  for (int c = tid; c < AT_ROWS * (AT_D / 8); c += 256) {
    const int r = c / (AT_D / 8), dc = c % (AT_D / 8);
    uint4 val = make_uint4(0, 0, 0, 0);
    if (r < rows) {
      const int hr = r / QB, i = r % QB, h = kvh * a.n_rep + hr;
      val = *reinterpret_cast<const uint4*>(a.q + (((size_t)b * a.T + q0 + i) * a.Hq + h) * AT_D + dc * 8);
    }
    *reinterpret_cast<uint4*>(k_lds + r * AT_KROW + dc * 16) = val;
  }
  __syncthreads();
  bf16x8 qB[2][8];
#pragma unroll
  for (int r2 = 0; r2 < 2; ++r2)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qB[r2][s] = *reinterpret_cast<const bf16x8*>(k_lds + (16 * r2 + l16) * AT_KROW + (32 * s + 8 * g4) * 2);
  __syncthreads();

  // query positions of the S rows this lane touches
  const int qpos_s0 = L - a.T + q0 + l16 % QB;
  const int qpos_s1 = L - a.T + q0 + (16 + l16) % QB;

  const uint16_t* Kb = a.kc + (size_t)b * a.seq_stride + (size_t)kvh * a.head_stride;
  const uint16_t* Vb = a.vc + (size_t)b * a.seq_stride + (size_t)kvh * a.head_stride;
  const int s_begin = split * a.chunk;
  const int s_end = min(L, s_begin + a.chunk);
  const int nblocks = (s_end - s_begin + AT_BLOCK - 1) / AT_BLOCK;

  // coalesced 16 B chunks of the K and V block rows (streaming loads), zero
  // outside the split; the next block is in flight while this one is computed
  uint4 kpre[8], vpre[8];
  auto load_block = [&](int key0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = i * 256 + tid, key = key0 + (c >> 5), dc = c & 31;
      const bool in = key < s_end;
      kpre[i] = in ? load_nt(Kb + (size_t)key * AT_D + dc * 8) : make_uint4(0, 0, 0, 0);
      vpre[i] = in ? load_nt(Vb + (size_t)key * AT_D + dc * 8) : make_uint4(0, 0, 0, 0);
    }
  };

  f32x16 O[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[mt][r] = 0.f;
  float m_s[2] = {-INFINITY, -INFINITY}, l_s[2] = {0.f, 0.f}, m_o = -INFINITY;

  load_block(s_begin);
  for (int blk = 0; blk < nblocks; ++blk) {
    const int key0 = s_begin + blk * AT_BLOCK;
    // 1. stage this block, then start the next block's loads
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = i * 256 + tid, off = (c >> 5) * AT_KROW + (c & 31) * 16;
      *reinterpret_cast<uint4*>(k_lds + off) = kpre[i];
      *reinterpret_cast<uint4*>(v_lds + off) = vpre[i];
    }
    lds_barrier();
    if (blk + 1 < nblocks) load_block(key0 + AT_BLOCK);

    // 2. S^T for keys [16 w, 16 w + 16) x rows [0, 32)
    f32x4 S[2];
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2)
#pragma unroll
      for (int j = 0; j < 4; ++j) S[r2][j] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8 kA = *reinterpret_cast<const bf16x8*>(k_lds + (16 * wave + l16) * AT_KROW + (32 * s + 8 * g4) * 2);
      S[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, qB[0][s], S[0], 0, 0, 0);
      S[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, qB[1][s], S[1], 0, 0, 0);
    }
    // 3. mask (key inside the split and <= the row's query position); row maxima
    float mx[2];
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int qp = r2 ? qpos_s1 : qpos_s0;
      const int kbase = key0 + 16 * wave + 4 * g4;
      const int lim = min(s_end - 1, qp) - kbase;   // keys kbase + j allowed iff j <= lim
      mx[r2] = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        S[r2][j] = j <= lim ? S[r2][j] : -INFINITY;
        mx[r2] = fmaxf(mx[r2], S[r2][j]);
      }
      mx[r2] = fmaxf(mx[r2], __shfl_xor(mx[r2], 16, 64));
      mx[r2] = fmaxf(mx[r2], __shfl_xor(mx[r2], 32, 64));
      if (lane < 16) m_lds[wave * AT_ROWS + 16 * r2 + lane] = mx[r2];
    }
    lds_barrier();
    // 4. common running max, probabilities, P^T to LDS
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int row = 16 * r2 + l16;
      const float mb = fmaxf(fmaxf(m_lds[row], m_lds[AT_ROWS + row]),
                             fmaxf(m_lds[2 * AT_ROWS + row], m_lds[3 * AT_ROWS + row]));
      const float mn = fmaxf(m_s[r2], mb);
      const bool live = mn != -INFINITY;
      const float alpha = live ? fast_exp2((m_s[r2] - mn) * a.cl2) : 1.f;
      const float base = live ? mn * a.cl2 : 0.f;
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) p[j] = fast_exp2(__builtin_fmaf(S[r2][j], a.cl2, -base));
      l_s[r2] = l_s[r2] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
      m_s[r2] = mn;
      const uint32_t lo = (uint32_t)f32_to_bf16(p[0]) | ((uint32_t)f32_to_bf16(p[1]) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(p[2]) | ((uint32_t)f32_to_bf16(p[3]) << 16);
      *reinterpret_cast<uint2*>(p_lds + row * AT_PROW + (16 * wave + 4 * g4) * 2) = make_uint2(lo, hi);
    }
    {
      const float mb = fmaxf(fmaxf(m_lds[l32], m_lds[AT_ROWS + l32]),
                             fmaxf(m_lds[2 * AT_ROWS + l32], m_lds[3 * AT_ROWS + l32]));
      const float mn = fmaxf(m_o, mb);
      const float alpha = mn == -INFINITY ? 1.f : fast_exp2((m_o - mn) * a.cl2);
      m_o = mn;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) O[mt] *= alpha;
    }
    lds_barrier();
    // 5. O^T[64 w .. 64 w + 64) += V^T P^T over the 64 keys
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 pB = *reinterpret_cast<const bf16x8*>(p_lds + l32 * AT_PROW + (16 * ks + 8 * h2) * 2);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const unsigned char* vcol = v_lds + (16 * ks + 8 * h2) * AT_KROW + (64 * wave + 32 * mt + l32) * 2;
        bf16x8 vA;
#pragma unroll
        for (int e = 0; e < 8; ++e) vA[e] = *reinterpret_cast<const __bf16*>(vcol + e * AT_KROW);
        O[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vA, pB, O[mt], 0, 0, 0);
      }
    }
    lds_barrier();
  }

  // ---- row sums: lanes sharing a row, then waves ----
#pragma unroll
  for (int r2 = 0; r2 < 2; ++r2) {
    float l = l_s[r2];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (lane < 16) l_lds[wave * AT_ROWS + 16 * r2 + lane] = l;
  }
  // O^T -> LDS as O[row][d] (reusing the K block region)
  float* o_lds = reinterpret_cast<float*>(k_lds);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 64 * wave + 32 * mt + 8 * (r >> 2) + 4 * h2 + (r & 3);
      o_lds[l32 * AT_OROW + d] = O[mt][r];
    }
  if (h2 == 0 && wave == 0) m_lds[l32] = m_o;
  __syncthreads();
  const bool single = nsplit == 1;
  if (single) {
    for (int idx = tid; idx < rows * AT_D; idx += 256) {
      const int r = idx / AT_D, d = idx % AT_D;
      float l = 0.f;
#pragma unroll
      for (int w = 0; w < AT_WAVES; ++w) l += l_lds[w * AT_ROWS + r];
      const int hr = r / QB, i = r % QB, h = kvh * a.n_rep + hr;
      const size_t o = ((size_t)b * a.T + q0 + i) * a.Hq * AT_D + (size_t)h * AT_D + d;
      float val = l > 0.f ? o_lds[r * AT_OROW + d] / l : 0.f;
      if (a.gate) val *= sigmoidf_(bf16_to_f32(a.gate[o]));
      a.out[o] = f32_to_bf16(val);
    }
  } else {
    float* part = a.ws + ((((size_t)b * a.Hkv + kvh) * a.qblocks + qb) * a.max_splits + split) * AT_PART;
    if (tid < AT_ROWS) {
      float l = 0.f;
#pragma unroll
      for (int w = 0; w < AT_WAVES; ++w) l += l_lds[w * AT_ROWS + tid];
      part[tid] = m_lds[tid];
      part[AT_ROWS + tid] = l;
    }
    for (int idx = tid; idx < rows * AT_D; idx += 256)
      part[2 * AT_ROWS + idx] = o_lds[(idx / AT_D) * AT_OROW + idx % AT_D];
  }
}

// Merge the split partials of one (row, KV head x query block, sequence) and apply
// the gate: thread d owns output column d; split weights exp(m_s - M) live in LDS.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  extern __shared__ float wsc[];  // max_splits weights
  __shared__ float red[8];
  const int r = blockIdx.x;
  const int kvh = blockIdx.y / a.qblocks, qb = blockIdx.y % a.qblocks;
  const int b = blockIdx.z;
  const int L = min(max(a.kv_len[b], 0), a.max_len);
  const int nsplit = (L + a.chunk - 1) / a.chunk;
  if (nsplit <= 1) return;  // finished in the main kernel
  const int q0 = qb * a.QB;
  const int QB = min(a.QB, a.T - q0);
  if (r >= a.n_rep * QB) return;
  const float* base = a.ws + (((size_t)b * a.Hkv + kvh) * a.qblocks + qb) * a.max_splits * AT_PART;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float m = -INFINITY;
  for (int s = tid; s < nsplit; s += 256) m = fmaxf(m, base[(size_t)s * AT_PART + r]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.f;
  for (int s = tid; s < nsplit; s += 256) {
    const float ms = base[(size_t)s * AT_PART + r];
    const float w = ms == -INFINITY ? 0.f : fast_exp2((ms - M) * a.cl2);
    wsc[s] = w;
    l += base[(size_t)s * AT_PART + AT_ROWS + r] * w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
  if (lane == 0) red[4 + wave] = l;
  __syncthreads();
  const float lsum = red[4] + red[5] + red[6] + red[7];
  const float* col = base + 2 * AT_ROWS + r * AT_D + tid;
  float acc = 0.f;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) acc += col[(size_t)s * AT_PART] * wsc[s];
  const int hr = r / QB, i = r % QB, h = kvh * a.n_rep + hr;
  const size_t o = ((size_t)b * a.T + q0 + i) * a.Hq * AT_D + (size_t)h * AT_D + tid;
  float val = lsum > 0.f ? acc / lsum : 0.f;
  if (a.gate) val *= sigmoidf_(bf16_to_f32(a.gate[o]));
  a.out[o] = f32_to_bf16(val);
}

static size_t attn_lds_bytes() { return AT_LDS_BYTES; }

}  // namespace lollm

using namespace lollm;

static int attn_geometry(int T, int Hq, int Hkv, int D, int max_len, int chunk, int* n_rep,
                         int* QB, int* qblocks, int* max_splits) {
  if (T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || max_len <= 0) return LOLLM_EINVAL;
  if (D != AT_D) return LOLLM_EUNSUPPORTED;
  if (chunk <= 0 || chunk % AT_BLOCK) return LOLLM_EINVAL;
  *n_rep = Hq / Hkv;
  if (*n_rep > AT_ROWS) return LOLLM_EUNSUPPORTED;
  *QB = AT_ROWS / *n_rep < T ? AT_ROWS / *n_rep : T;
  *qblocks = (T + *QB - 1) / *QB;
  *max_splits = (max_len + chunk - 1) / chunk;
  return LOLLM_OK;
}

LOLLM_API long long lollm_attn_workspace_bytes(int B, int T, int Hq, int Hkv, int D,
                                               int max_len, int chunk) {
  int n_rep, QB, qblocks, max_splits;
  if (B <= 0) return -1;
  if (attn_geometry(T, Hq, Hkv, D, max_len, chunk, &n_rep, &QB, &qblocks, &max_splits))
    return -1;
  return (long long)B * Hkv * qblocks * max_splits * AT_PART * sizeof(float);
}

LOLLM_API int lollm_attn_verify(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* kv_len, const void* gate, void* out,
                                void* workspace, long long workspace_bytes, int B, int T, int Hq,
                                int Hkv, int D, int max_len, long long seq_stride,
                                long long head_stride, int chunk, float scale, void* stream) {
  if (!q || !k_cache || !v_cache || !kv_len || !out || B <= 0) return LOLLM_EINVAL;
  int n_rep, QB, qblocks, max_splits;
  int rc = attn_geometry(T, Hq, Hkv, D, max_len, chunk, &n_rep, &QB, &qblocks, &max_splits);
  if (rc) return rc;
  if (head_stride < (long long)max_len * D || seq_stride < head_stride * Hkv) return LOLLM_EINVAL;
  if (head_stride % 8 || seq_stride % 8) return LOLLM_EINVAL;  // 16-byte aligned rows
  const long long need = (long long)B * Hkv * qblocks * max_splits * AT_PART * sizeof(float);
  if (max_splits > 1 && (!workspace || workspace_bytes < need)) return LOLLM_EINVAL;
  if (max_splits > 16384) return LOLLM_EUNSUPPORTED;
  AttnArgs a;
  a.q = (const uint16_t*)q; a.kc = (const uint16_t*)k_cache; a.vc = (const uint16_t*)v_cache;
  a.kv_len = kv_len; a.gate = (const uint16_t*)gate; a.out = (uint16_t*)out;
  a.ws = (float*)workspace; a.seq_stride = seq_stride; a.head_stride = head_stride;
  a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.n_rep = n_rep; a.QB = QB; a.qblocks = qblocks;
  a.chunk = chunk; a.max_splits = max_splits; a.max_len = max_len;
  a.cl2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  static bool lds_set = false;
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute((const void*)attn_verify_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)attn_lds_bytes());
    if (e != hipSuccess) return LOLLM_EHIP_BASE + (int)e;
    lds_set = true;
  }
  dim3 grid(max_splits, Hkv * qblocks, B);
  hipLaunchKernelGGL(attn_verify_kernel, grid, dim3(256), attn_lds_bytes(), st, a);
  if ((rc = launch_status())) return rc;
  if (max_splits > 1) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3(AT_ROWS, Hkv * qblocks, B), dim3(256),
                       (size_t)max_splits * sizeof(float), st, a);
    rc = launch_status();
  }
  return rc;
}

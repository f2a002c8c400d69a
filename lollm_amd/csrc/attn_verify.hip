// Gated GQA attention over a per-sequence KV cache for the 1 + k verify block
// (gfx950, bf16 MFMA).
//
// Math (src/qwen3_5/blocks.py:226-235 + src/attention.py:43-51): query i of the T
// new positions of sequence b sits at absolute position L_b - T + i and attends the
// keys at positions <= that (offset-causal; plain causal when T == L_b); scores are
// scaled by D^-0.5; q-head h reads KV head h / n_rep (blocks.py:152-156, no
// expansion is materialised); the output is o * sigmoid(gate) (blocks.py:235).
//
// Work decomposition (balanced split-K).  A "pair" is (sequence b, KV head x query
// block); its 32 MFMA rows pack n_rep q-heads x QB queries, so every K/V byte read
// from HBM serves all the q-heads that share it.  A pair's context is cut into
// 64-key blocks, and the blocks of all pairs, laid end to end (pair-major), are dealt
// out in equal contiguous ranges to a fixed grid of workgroups sized to the GPU
// (two per CU).  Every workgroup therefore streams the same number of bytes whatever
// the context lengths, and no CU idles while another finishes a long sequence.  A
// range cut inside a pair yields a partial (m, l, O) per piece; a combine kernel
// merges the pieces of the pairs that were cut and applies the gate (a pair that one
// workgroup covers whole is finished in place).
//
// Inside a workgroup (4 waves) each 64-key block is:
//   - staged in LDS from registers filled by coalesced 16-byte streaming loads; the
//     next block's loads (possibly of the next pair) are issued right after staging,
//     so they are in flight while this block is computed; barriers order LDS only;
//   - S^T for keys [16w, 16w+16) x 32 rows on wave w (16x16x32 MFMA, K from LDS,
//     Q^T in registers, loaded once per pair straight from global memory); masked
//     row maxima exchanged through LDS so all waves share one running max; P^T to
//     LDS as bf16;
//   - O^T[64w, 64w+64) += V^T P^T on wave w (32x32x16 MFMA, A = V^T read from LDS).
#include "common.h"

namespace lollm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AT_D = 256;            // head dim
constexpr int AT_ROWS = 32;          // MFMA rows per pair (n_rep x QB)
constexpr int AT_BLOCK = 64;         // keys per block
constexpr int AT_WAVES = 4;
constexpr int AT_MAXB = 512;         // sequences per call (prefix table in LDS)
constexpr int AT_KROW = AT_D * 2 + 16;        // padded bytes per K / V row in LDS
constexpr int AT_PROW = AT_BLOCK * 2 + 16;    // padded bytes per P^T row in LDS
constexpr int AT_OROW = AT_D + 1;             // padded floats per O row in LDS
constexpr int AT_PART = 2 * AT_ROWS + AT_ROWS * AT_D;  // floats per partial
constexpr int AT_LDS_K = 0;
constexpr int AT_LDS_V = AT_LDS_K + AT_BLOCK * AT_KROW;
constexpr int AT_LDS_P = AT_LDS_V + AT_BLOCK * AT_KROW;
constexpr int AT_LDS_M = AT_LDS_P + AT_ROWS * AT_PROW;
constexpr int AT_LDS_PRE = AT_LDS_M + 2 * AT_WAVES * AT_ROWS * 4;
constexpr int AT_LDS_LEN = AT_LDS_PRE + (AT_MAXB + 1) * 4;
constexpr int AT_LDS_BYTES = AT_LDS_LEN + AT_MAXB * 4 + 64;

struct AttnArgs {
  const uint16_t* q;       // (B, T, Hq, D)
  const uint16_t* kc;      // K cache
  const uint16_t* vc;      // V cache
  const int32_t* kv_len;   // (B) keys per sequence, the T new ones included
  const uint16_t* gate;    // (B, T, Hq * D) or null
  uint16_t* out;           // (B, T, Hq * D)
  float* ws;               // partials: (nw + pairs) x AT_PART
  long long seq_stride, head_stride;  // cache strides in elements
  int B, T, Hq, Hkv, n_rep, QB, qblocks, max_len, nw;
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

__device__ __forceinline__ int seq_len(const AttnArgs& a, int b) {
  return min(max(a.kv_len[b], 0), a.max_len);  // never past the cache capacity
}

__device__ __forceinline__ int nblk_of(int L) { return (L + AT_BLOCK - 1) / AT_BLOCK; }

// pre[b] = blocks of sequences 0..b-1 (pre[0] = 0), for b = 0..B, and len[b] = the
// clamped key count of sequence b, built in LDS by the whole workgroup (so the main
// loop never waits on a global load to address the next block).  Returns pre[B].
__device__ int build_prefix(const AttnArgs& a, int* pre, int* len, int* tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int carry = 0;
  if (tid == 0) pre[0] = 0;
  for (int base = 0; base < a.B; base += 256) {
    const int b = base + tid;
    const int Lb = b < a.B ? seq_len(a, b) : 0;
    if (b < a.B) len[b] = Lb;
    int v = nblk_of(Lb);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(v, d, 64);
      if (lane >= d) v += o;
    }
    if (lane == 63) tmp[wave] = v;
    __syncthreads();
    int before = carry, all = carry;
#pragma unroll
    for (int w = 0; w < AT_WAVES; ++w) {
      if (w < wave) before += tmp[w];
      all += tmp[w];
    }
    if (b < a.B) pre[b + 1] = before + v;
    carry = all;
    __syncthreads();
  }
  return carry;
}

// First unit of workgroup w and the workgroup that owns unit u, for U units dealt
// out to nw workgroups in equal contiguous ranges: w owns [U w / nw, U (w+1) / nw).
__device__ __forceinline__ long long unit_begin(long long U, int w, int nw) {
  return U * w / nw;
}
__device__ __forceinline__ int unit_owner(long long U, long long u, int nw) {
  return (int)(((u + 1) * nw - 1) / U);
}

__global__ __launch_bounds__(256, 2) void attn_verify_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* k_lds = smem + AT_LDS_K;
  unsigned char* v_lds = smem + AT_LDS_V;
  unsigned char* p_lds = smem + AT_LDS_P;
  float* m_lds = reinterpret_cast<float*>(smem + AT_LDS_M);    // [wave][row]
  float* l_lds = m_lds + AT_WAVES * AT_ROWS;
  int* pre = reinterpret_cast<int*>(smem + AT_LDS_PRE);
  int* len = reinterpret_cast<int*>(smem + AT_LDS_LEN);
  int* tmp = len + AT_MAXB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4, l32 = lane & 31, h2 = lane >> 5;
  const int w = blockIdx.x;
  const int PH = a.Hkv * a.qblocks;  // pairs per sequence

  const long long U = (long long)PH * build_prefix(a, pre, len, tmp);
  const long long u0 = unit_begin(U, w, a.nw), u1 = unit_begin(U, w + 1, a.nw);
  if (u0 >= u1) return;

  // locate the first unit: the last sequence whose first unit is <= u0 (never empty)
  int b;
  {
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((long long)PH * pre[mid] <= u0) lo = mid; else hi = mid - 1;
    }
    b = lo;
  }
  int nb = pre[b + 1] - pre[b];
  int ph, j;
  {
    const long long r = u0 - (long long)PH * pre[b];
    ph = (int)(r / nb);
    j = (int)(r % nb);
  }

  // Block jj of pair (bb, pp): coalesced 16 B streaming loads.  Keys past the
  // sequence's last one read its last key (in bounds) and are zeroed, branch-free.
  uint4 kpre[8], vpre[8];
  auto load_block = [&](int bb, int pp, int jj) {
    const int kvh = pp / a.qblocks;
    const int Lb = len[bb];
    const uint16_t* Kb = a.kc + (size_t)bb * a.seq_stride + (size_t)kvh * a.head_stride;
    const uint16_t* Vb = a.vc + (size_t)bb * a.seq_stride + (size_t)kvh * a.head_stride;
    const int key0 = jj * AT_BLOCK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = i * 256 + tid, key = key0 + (c >> 5), dc = c & 31;
      const size_t off = (size_t)min(key, Lb - 1) * AT_D + dc * 8;
      kpre[i] = load_nt(Kb + off);
      vpre[i] = load_nt(Vb + off);
    }
  };
  auto zero_tail = [&](int Lb, int jj) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = jj * AT_BLOCK + ((i * 256 + tid) >> 5);
      if (key >= Lb) { kpre[i] = make_uint4(0, 0, 0, 0); vpre[i] = make_uint4(0, 0, 0, 0); }
    }
  };
  // Q^T of pair (bb, pp) straight into the MFMA B operands (rows r = hr * QB + i)
  bf16x8 qB[2][8];
  auto load_q = [&](int bb, int pp) {
    const int kvh = pp / a.qblocks, qb = pp % a.qblocks;
    const int q0_ = qb * a.QB, QB_ = min(a.QB, a.T - q0_), rows_ = a.n_rep * QB_;
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int r = 16 * r2 + l16;
      const bool live = r < rows_;
      const int hr = live ? r / QB_ : 0, i = live ? r % QB_ : 0, h = kvh * a.n_rep + hr;
      const uint16_t* qrow = a.q + (((size_t)bb * a.T + q0_ + i) * a.Hq + h) * AT_D + 8 * g4;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * s);
        qB[r2][s] = __builtin_bit_cast(bf16x8, live ? v : make_uint4(0, 0, 0, 0));
      }
    }
  };

  f32x16 O[2];
  float m_s[2], l_s[2], m_o;
  int qpos_s0 = 0, qpos_s1 = 0, L = 0, QB = 1, q0 = 0, rows = 0, j_first = 0;

  load_block(b, ph, j);
  load_q(b, ph);
  for (long long u = u0; u < u1; ++u) {
    const bool seg_first = (u == u0) || (j == 0);
    const bool seg_last = (u == u1 - 1) || (j == nb - 1);
    const int kvh = ph / a.qblocks, qb = ph % a.qblocks;
    if (seg_first) {
      L = len[b];
      q0 = qb * a.QB;
      QB = min(a.QB, a.T - q0);
      rows = a.n_rep * QB;
      j_first = j;
      qpos_s0 = L - a.T + q0 + l16 % QB;
      qpos_s1 = L - a.T + q0 + (16 + l16) % QB;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[mt][r] = 0.f;
      m_s[0] = m_s[1] = -INFINITY;
      l_s[0] = l_s[1] = 0.f;
      m_o = -INFINITY;
    }
    const int key0 = j * AT_BLOCK;

    // 1. stage this block, then start the next unit's loads
    zero_tail(L, j);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = i * 256 + tid, off = (c >> 5) * AT_KROW + (c & 31) * 16;
      *reinterpret_cast<uint4*>(k_lds + off) = kpre[i];
      *reinterpret_cast<uint4*>(v_lds + off) = vpre[i];
    }
    lds_barrier();
    int nb_b = b, nb_ph = ph, nb_j = j + 1, nb_nb = nb;
    if (nb_j == nb) {
      nb_j = 0;
      if (++nb_ph == PH) {
        nb_ph = 0;
        do { ++nb_b; } while (nb_b < a.B && pre[nb_b + 1] == pre[nb_b]);
        if (nb_b < a.B) nb_nb = pre[nb_b + 1] - pre[nb_b];
      }
    }
    const bool more = u + 1 < u1;
    if (more) load_block(nb_b, nb_ph, nb_j);

    // 2. S^T for keys [16 w, 16 w + 16) x rows [0, 32)
    f32x4 S[2];
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) S[r2][jj] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8 kA = *reinterpret_cast<const bf16x8*>(k_lds + (16 * wave + l16) * AT_KROW + (32 * s + 8 * g4) * 2);
      S[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, qB[0][s], S[0], 0, 0, 0);
      S[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, qB[1][s], S[1], 0, 0, 0);
    }
    // the next unit starts a new pair: its Q is in flight while this block finishes
    if (seg_last && more) load_q(nb_b, nb_ph);
    // 3. mask (key < L and <= the row's query position); row maxima
    float mx[2];
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int qp = r2 ? qpos_s1 : qpos_s0;
      const int kbase = key0 + 16 * wave + 4 * g4;
      const int lim = min(L - 1, qp) - kbase;   // keys kbase + jj allowed iff jj <= lim
      mx[r2] = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        S[r2][jj] = jj <= lim ? S[r2][jj] : -INFINITY;
        mx[r2] = fmaxf(mx[r2], S[r2][jj]);
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
      for (int jj = 0; jj < 4; ++jj) p[jj] = fast_exp2(__builtin_fmaf(S[r2][jj], a.cl2, -base));
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

    if (seg_last) {
      // ---- row sums: lanes sharing a row, then waves ----
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        float l = l_s[r2];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (lane < 16) l_lds[wave * AT_ROWS + 16 * r2 + lane] = l;
      }
      // O^T -> LDS as O[row][d] (the K block region is free until the next staging)
      float* o_lds = reinterpret_cast<float*>(k_lds);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = 64 * wave + 32 * mt + 8 * (r >> 2) + 4 * h2 + (r & 3);
          o_lds[l32 * AT_OROW + d] = O[mt][r];
        }
      if (h2 == 0 && wave == 0) m_lds[l32] = m_o;
      lds_barrier();
      const int pair = b * PH + ph;
      if (j_first == 0 && j == nb - 1) {
        // the whole pair in this workgroup: finish in place, 8 columns per thread
#pragma unroll 1
        for (int it = 0; it < 4; ++it) {
          const int c = it * 256 + tid, r = c >> 5, d0 = (c & 31) * 8;
          if (r >= rows) continue;
          const int hr = r / QB, i = r % QB, h = kvh * a.n_rep + hr;
          const size_t ob = ((size_t)b * a.T + q0 + i) * a.Hq * AT_D + (size_t)h * AT_D + d0;
          const uint4 gv = a.gate ? *reinterpret_cast<const uint4*>(a.gate + ob) : make_uint4(0, 0, 0, 0);
          float l = 0.f;
#pragma unroll
          for (int ww = 0; ww < AT_WAVES; ++ww) l += l_lds[ww * AT_ROWS + r];
          const float inv = l > 0.f ? 1.f / l : 0.f;
          const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
          uint32_t ow[4];
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            float y[2];
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
              float val = o_lds[r * AT_OROW + d0 + e + t2] * inv;
              if (a.gate) val *= sigmoidf_(bf16_to_f32((uint16_t)(gw[e >> 1] >> (16 * t2))));
              y[t2] = val;
            }
            ow[e >> 1] = (uint32_t)f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16);
          }
          *reinterpret_cast<uint4*>(a.out + ob) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        }
      } else {
        // one piece of a pair cut between workgroups: slot w + pair is unique
        // (pieces are ordered in both w and pair)
        float* part = a.ws + ((size_t)w + pair) * AT_PART;
        if (tid < AT_ROWS) {
          float l = 0.f;
#pragma unroll
          for (int ww = 0; ww < AT_WAVES; ++ww) l += l_lds[ww * AT_ROWS + tid];
          part[tid] = m_lds[tid];
          part[AT_ROWS + tid] = l;
        }
        for (int c = tid; c < rows * (AT_D / 4); c += 256) {
          const int r = c / (AT_D / 4), d0 = (c % (AT_D / 4)) * 4;
          const float* src = o_lds + r * AT_OROW + d0;
          *reinterpret_cast<float4*>(part + 2 * AT_ROWS + r * AT_D + d0) =
              make_float4(src[0], src[1], src[2], src[3]);
        }
      }
      lds_barrier();  // o_lds / l_lds / m_lds read before the next staging overwrites them
    }
    b = nb_b; ph = nb_ph; j = nb_j; nb = nb_nb;
  }
}

// Merge the pieces of pair blockIdx.y for row blockIdx.x and apply the gate: thread d
// owns output column d; piece weights exp(m_s - M) live in LDS.  Pairs finished by
// one workgroup are skipped; pairs with no keys get zeros.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  __shared__ float wsc[1024];   // piece weights (0 for workgroups with no units)
  __shared__ float lsc[1024];   // piece row sums
  __shared__ float red[8];
  __shared__ int sred[8];
  const int r = blockIdx.x, pair = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int PH = a.Hkv * a.qblocks;
  const int b = pair / PH, ph = pair % PH;
  const int kvh = ph / a.qblocks, qb = ph % a.qblocks;
  const int q0 = qb * a.QB;
  const int QB = min(a.QB, a.T - q0);
  if (r >= a.n_rep * QB) return;
  const int hr = r / QB, i = r % QB, h = kvh * a.n_rep + hr;
  const size_t o = ((size_t)b * a.T + q0 + i) * a.Hq * AT_D + (size_t)h * AT_D + tid;
  const float gl = a.gate ? bf16_to_f32(a.gate[o]) : 0.f;   // in flight from the start
  // blocks before sequence b, and in total
  int before = 0, total = 0;
  for (int s = tid; s < a.B; s += 256) {
    const int n = nblk_of(seq_len(a, s));
    total += n;
    if (s < b) before += n;
  }
#pragma unroll
  for (int of = 32; of > 0; of >>= 1) {
    before += __shfl_xor(before, of, 64);
    total += __shfl_xor(total, of, 64);
  }
  if (lane == 0) { sred[wave] = before; sred[4 + wave] = total; }
  __syncthreads();
  before = sred[0] + sred[1] + sred[2] + sred[3];
  total = sred[4] + sred[5] + sred[6] + sred[7];
  const int nb = nblk_of(seq_len(a, b));
  if (nb == 0) {
    a.out[o] = 0;
    return;
  }
  const long long U = (long long)PH * total;
  const long long first = (long long)PH * before + (long long)ph * nb;
  const int wf = unit_owner(U, first, a.nw), wl = unit_owner(U, first + nb - 1, a.nw);
  if (wf == wl) return;  // finished in the main kernel
  // pieces: slot w + pair of every workgroup w in [wf, wl] whose range is not empty
  // (with fewer blocks than workgroups, empty workgroups sit between the owners)
  const int np = wl - wf + 1;
  const float* base = a.ws + ((size_t)wf + pair) * AT_PART;
  float m = -INFINITY;
  for (int s = tid; s < np; s += 256) {
    const bool live = unit_begin(U, wf + s, a.nw) < unit_begin(U, wf + s + 1, a.nw);
    const float ms = live ? base[(size_t)s * AT_PART + r] : -INFINITY;
    lsc[s] = live ? base[(size_t)s * AT_PART + AT_ROWS + r] : 0.f;
    wsc[s] = ms;
    m = fmaxf(m, ms);
  }
#pragma unroll
  for (int of = 32; of > 0; of >>= 1) m = fmaxf(m, __shfl_xor(m, of, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.f;
  for (int s = tid; s < np; s += 256) {
    const float ms = wsc[s];
    const float wgt = ms == -INFINITY ? 0.f : fast_exp2((ms - M) * a.cl2);
    wsc[s] = wgt;
    l += lsc[s] * wgt;
  }
#pragma unroll
  for (int of = 32; of > 0; of >>= 1) l += __shfl_xor(l, of, 64);
  if (lane == 0) red[4 + wave] = l;
  __syncthreads();
  const float lsum = red[4] + red[5] + red[6] + red[7];
  const float* col = base + 2 * AT_ROWS + r * AT_D + tid;
  float acc = 0.f;
#pragma unroll 8
  for (int s = 0; s < np; ++s) {
    const float wgt = wsc[s];
    const float v = col[(size_t)s * AT_PART];   // in bounds for every slot; junk if dead
    acc += wgt != 0.f ? v * wgt : 0.f;
  }
  float val = lsum > 0.f ? acc / lsum : 0.f;
  if (a.gate) val *= sigmoidf_(gl);
  a.out[o] = f32_to_bf16(val);
}

}  // namespace lollm

using namespace lollm;

static int attn_geometry(int B, int T, int Hq, int Hkv, int D, int max_len, int* n_rep, int* QB,
                         int* qblocks) {
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || max_len <= 0) return LOLLM_EINVAL;
  if (D != AT_D) return LOLLM_EUNSUPPORTED;
  if (B > AT_MAXB) return LOLLM_EUNSUPPORTED;
  *n_rep = Hq / Hkv;
  if (*n_rep > AT_ROWS) return LOLLM_EUNSUPPORTED;
  *QB = AT_ROWS / *n_rep < T ? AT_ROWS / *n_rep : T;
  *qblocks = (T + *QB - 1) / *QB;
  return LOLLM_OK;
}

// Workgroups of the balanced grid: `grid` if positive, else two per CU of the
// current device.  A piece count per pair above the combine's table size is refused.
static int attn_grid(int grid) {
  if (grid > 0) return grid;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  return cus > 0 ? 2 * cus : -1;
}

LOLLM_API long long lollm_attn_workspace_bytes(int B, int T, int Hq, int Hkv, int D,
                                               int max_len, int grid) {
  int n_rep, QB, qblocks;
  if (attn_geometry(B, T, Hq, Hkv, D, max_len, &n_rep, &QB, &qblocks)) return -1;
  const int nw = attn_grid(grid);
  if (nw <= 0) return -1;
  return ((long long)nw + (long long)B * Hkv * qblocks) * AT_PART * (long long)sizeof(float);
}

LOLLM_API int lollm_attn_verify(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* kv_len, const void* gate, void* out,
                                void* workspace, long long workspace_bytes, int B, int T, int Hq,
                                int Hkv, int D, int max_len, long long seq_stride,
                                long long head_stride, int grid, float scale, void* stream) {
  if (!q || !k_cache || !v_cache || !kv_len || !out) return LOLLM_EINVAL;
  int n_rep, QB, qblocks;
  int rc = attn_geometry(B, T, Hq, Hkv, D, max_len, &n_rep, &QB, &qblocks);
  if (rc) return rc;
  if (grid < 0 || grid > 1024) return LOLLM_EINVAL;  // pieces per pair <= combine table
  if (head_stride < (long long)max_len * D || seq_stride < head_stride * Hkv) return LOLLM_EINVAL;
  if (head_stride % 8 || seq_stride % 8) return LOLLM_EINVAL;  // 16-byte aligned rows
  const int nw = attn_grid(grid);
  if (nw <= 0 || nw > 1024) return LOLLM_EUNSUPPORTED;
  const long long need = ((long long)nw + (long long)B * Hkv * qblocks) * AT_PART * (long long)sizeof(float);
  if (!workspace || workspace_bytes < need) return LOLLM_EINVAL;
  AttnArgs a;
  a.q = (const uint16_t*)q; a.kc = (const uint16_t*)k_cache; a.vc = (const uint16_t*)v_cache;
  a.kv_len = kv_len; a.gate = (const uint16_t*)gate; a.out = (uint16_t*)out;
  a.ws = (float*)workspace; a.seq_stride = seq_stride; a.head_stride = head_stride;
  a.B = B; a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.n_rep = n_rep; a.QB = QB; a.qblocks = qblocks;
  a.max_len = max_len; a.nw = nw;
  a.cl2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  static bool lds_set[64] = {};   // per device: the attribute is set on the current device
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return LOLLM_EUNSUPPORTED;
  if (!lds_set[dev]) {
    hipError_t e = hipFuncSetAttribute((const void*)attn_verify_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, AT_LDS_BYTES);
    if (e != hipSuccess) return LOLLM_EHIP_BASE + (int)e;
    lds_set[dev] = true;
  }
  hipLaunchKernelGGL(attn_verify_kernel, dim3(nw), dim3(256), AT_LDS_BYTES, st, a);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(AT_ROWS, B * Hkv * qblocks), dim3(256), 0, st, a);
  return launch_status();
}

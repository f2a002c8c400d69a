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
// 128-key blocks ("units"), and the units of all pairs, laid end to end (pair-major),
// are dealt out in equal contiguous ranges to a fixed grid of one 8-wave workgroup per
// CU.  Every workgroup therefore streams the same number of bytes whatever the context
// lengths, and no CU idles while another finishes a long sequence.  Each workgroup
// leaves one partial (m, l, O) per pair it touched; a combine kernel merges the pieces
// of every pair and applies the gate.
//
// Inside a workgroup, two units are in flight ahead of the one computed (256 KB per
// CU), all their loads issued unconditionally through buffer descriptors (a unit past
// the range reads through an empty descriptor: zeros, no traffic), so the compiler's
// vmcnt waits only ever wait for the unit about to be used:
//   - K: wave w loads its own 16 keys straight into the S MFMA A operand;
//   - V: coalesced non-temporal loads into registers, staged in LDS (padded rows);
//   - Q: one unit ahead, staged in LDS (two buffers) at the pair's first unit;
// and each unit is:
//   - S^T for keys [16w, 16w+16) x 32 rows on wave w (16x16x32 MFMA, Q^T from LDS);
//     P^T to LDS as bf16 against a per-row reference max shared by all waves, with the
//     masked row maxima to LDS, then one barrier: only when a block's maximum exceeds
//     the reference by 16 in the exponent (and at a pair's first block) do all waves
//     move the reference, rescale l and O and rewrite P^T behind a second barrier;
//   - O^T[32w, 32w+32) += V^T P^T on wave w (32x32x16 MFMA, A = V^T read from LDS).
#include "common.h"

namespace lollm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AT_D = 256;            // head dim
constexpr int AT_ROWS = 32;          // MFMA rows per pair (n_rep x QB)
constexpr int AT_BLOCK = 128;        // keys per block
constexpr int AT_WAVES = 8;
constexpr int AT_THREADS = 64 * AT_WAVES;
constexpr int AT_MAXB = 512;         // sequences per call (prefix table in LDS)
constexpr int AT_KROW = AT_D * 2 + 16;        // padded bytes per K / V row in LDS
constexpr int AT_PROW = AT_BLOCK * 2 + 16;    // padded bytes per P^T row in LDS
constexpr int AT_OROW = AT_D + 1;             // padded floats per O row in LDS
constexpr int AT_PART = 2 * AT_ROWS + AT_ROWS * AT_D;  // floats per partial
constexpr int AT_LDS_V = 0;                                 // V block; O at a pair's end
constexpr int AT_LDS_Q = AT_LDS_V + AT_BLOCK * AT_KROW;     // two Q buffers
constexpr int AT_LDS_P = AT_LDS_Q + 2 * AT_ROWS * AT_KROW;
constexpr int AT_LDS_M = AT_LDS_P + AT_ROWS * AT_PROW;
constexpr int AT_LDS_PRE = AT_LDS_M + 2 * AT_WAVES * AT_ROWS * 4;
constexpr int AT_LDS_LEN = AT_LDS_PRE + (AT_MAXB + 1) * 4;
constexpr int AT_LDS_BYTES = AT_LDS_LEN + AT_MAXB * 4 + 64;
static_assert(AT_ROWS * AT_OROW * 4 <= AT_BLOCK * AT_KROW, "O of a pair is staged in the V region");
static_assert(AT_LDS_BYTES <= 160 * 1024, "one workgroup per CU");

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
  for (int base = 0; base < a.B; base += AT_THREADS) {
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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t at_rsrc(const void* base, uint32_t bytes) {
  return buf_rsrc(base, bytes);
}
// AUX = 2: the non-temporal hint (K and V are read once per launch and should not
// displace reusable lines; measured 9% faster than the default policy on the C3 shape)
template <int AUX>
__device__ __forceinline__ u32x4_t at_bload(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, AUX));
}

// Position of a unit in the pair-major block order: sequence b, pair ph of it, block j
// of the pair's nb blocks.
struct AtCursor {
  int b, ph, j, nb;
};

__global__ __launch_bounds__(AT_THREADS, 1) void attn_verify_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* v_lds = smem + AT_LDS_V;
  unsigned char* q_lds = smem + AT_LDS_Q;   // two buffers of AT_ROWS rows
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
  {
    // the combine's table: per pair, the first and last workgroup whose range touches it
    // (-1 for a pair with no keys) and the unit count, so the combine reads one entry
    // instead of rebuilding the block prefix
    const int npairs = a.B * PH;
    int4* tab = reinterpret_cast<int4*>(a.ws + (size_t)(a.nw + npairs) * AT_PART);
    for (int p = w * AT_THREADS + tid; p < npairs; p += a.nw * AT_THREADS) {
      const int pb = p / PH, pph = p % PH, pnb = pre[pb + 1] - pre[pb];
      int wf = -1, wl = -1;
      if (pnb > 0) {
        const long long first = (long long)PH * pre[pb] + (long long)pph * pnb;
        wf = unit_owner(U, first, a.nw);
        wl = unit_owner(U, first + pnb - 1, a.nw);
      }
      tab[p] = make_int4(wf, wl, (int)(uint32_t)U, (int)(uint32_t)(U >> 32));
    }
  }
  const long long u0 = unit_begin(U, w, a.nw), u1 = unit_begin(U, w + 1, a.nw);
  if (u0 >= u1) return;

  // locate the first unit: the last sequence whose first unit is <= u0 (never empty)
  AtCursor C;
  {
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((long long)PH * pre[mid] <= u0) lo = mid; else hi = mid - 1;
    }
    C.b = lo;
    C.nb = pre[C.b + 1] - pre[C.b];
    const long long r = u0 - (long long)PH * pre[C.b];
    C.ph = (int)(r / C.nb);
    C.j = (int)(r % C.nb);
  }
  // (cursor fields are the same in every lane: kept in scalar registers)
  auto uni = [](AtCursor X) {
    X.b = __builtin_amdgcn_readfirstlane(X.b);
    X.ph = __builtin_amdgcn_readfirstlane(X.ph);
    X.j = __builtin_amdgcn_readfirstlane(X.j);
    X.nb = __builtin_amdgcn_readfirstlane(X.nb);
    return X;
  };
  C = uni(C);
  auto advance = [&](const AtCursor& X) {
    AtCursor Y = X;
    if (Y.b >= a.B) return Y;
    if (++Y.j == Y.nb) {
      Y.j = 0;
      if (++Y.ph == PH) {
        Y.ph = 0;
        do { ++Y.b; } while (Y.b < a.B && pre[Y.b + 1] == pre[Y.b]);
        if (Y.b < a.B) Y.nb = pre[Y.b + 1] - pre[Y.b];
      }
    }
    return uni(Y);
  };

  // The loads of a unit (all unconditional: a unit past the range, or Q of a unit that
  // does not start its pair, gets an empty descriptor and reads zeros without traffic).
  //   V: cooperative, chunk c = 512 i + tid holds key 16 i + tid / 32, bytes 16 (tid % 32)
  //   K: wave w's own 16 keys straight into the S MFMA A operand (lane: key 16 w + l16,
  //      bytes 64 s + 16 g4 for k-step s); keys past the sequence read zero.  Default
  //      cache policy: each load reads half of 16 lines, and L2 merges the two halves
  //      (with the non-temporal hint they were fetched separately: 10% slower)
  //   Q: cooperative rows r = 16 it + tid / 32 (r = hr QB + i), staged at the pair's start;
  //      one unit ahead, issued first in its unit's loads so waiting for it never waits
  //      for the later K/V loads
  u32x4_t vr[2][8], kr[2][8], qr[2];
  auto issue_v = [&](int set, const AtCursor& X, bool live) {
    const int kvh = live ? X.ph / a.qblocks : 0;
    const uint32_t bytes = live ? (uint32_t)__builtin_amdgcn_readfirstlane(len[X.b]) * (AT_D * 2) : 0u;
    const uint16_t* base = a.vc + (live ? (size_t)X.b * a.seq_stride + (size_t)kvh * a.head_stride : 0);
    const __amdgpu_buffer_rsrc_t rs = at_rsrc(base, bytes);
    const uint32_t vo = (uint32_t)(X.j * AT_BLOCK + (tid >> 5)) * (AT_D * 2) + (uint32_t)(tid & 31) * 16u;
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[set][i] = at_bload<2>(rs, vo, (uint32_t)i * 16u * (AT_D * 2));
  };
  auto issue_k = [&](int set, const AtCursor& X, bool live) {
    const int kvh = live ? X.ph / a.qblocks : 0;
    const uint32_t bytes = live ? (uint32_t)__builtin_amdgcn_readfirstlane(len[X.b]) * (AT_D * 2) : 0u;
    const uint16_t* base = a.kc + (live ? (size_t)X.b * a.seq_stride + (size_t)kvh * a.head_stride : 0);
    const __amdgpu_buffer_rsrc_t rs = at_rsrc(base, bytes);
    const uint32_t ko = (uint32_t)(X.j * AT_BLOCK + 16 * wave + l16) * (AT_D * 2) + (uint32_t)g4 * 16u;
#pragma unroll
    for (int s = 0; s < 8; ++s) kr[set][s] = at_bload<0>(rs, ko + (uint32_t)s * 64u, 0u);
  };
  auto issue_q = [&](const AtCursor& X, bool load) {
    const int kvh = load ? X.ph / a.qblocks : 0, qb = load ? X.ph % a.qblocks : 0;
    const int q0_ = qb * a.QB, QB_ = min(a.QB, a.T - q0_), rows_ = a.n_rep * QB_;
    const uint32_t bytes = load ? (uint32_t)a.T * (uint32_t)a.Hq * (AT_D * 2) : 0u;
    const uint16_t* base = a.q + (load ? (size_t)X.b * a.T * a.Hq * AT_D : 0);
    const __amdgpu_buffer_rsrc_t rs = at_rsrc(base, bytes);
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int r = 16 * it + (tid >> 5);
      const int hr = r / QB_, i = r % QB_;
      const uint32_t qo = r < rows_ ? ((uint32_t)(q0_ + i) * (uint32_t)a.Hq + (uint32_t)(kvh * a.n_rep + hr)) *
                                          (AT_D * 2) + (uint32_t)(tid & 31) * 16u
                                    : 0xFFFFFFF0u;
      qr[it] = at_bload<0>(rs, qo, 0u);
    }
  };

  AtCursor X1 = advance(C), X2 = advance(X1);
  issue_q(C, true);
  issue_v(0, C, true);
  issue_k(0, C, true);
  issue_v(1, X1, u0 + 1 < u1);
  issue_k(1, X1, u0 + 1 < u1);

  f32x16 O;   // O^T of this wave's 32 value columns
  float m_s[2], l_s[2], m_o;
  int qpos_s0 = 0, qpos_s1 = 0, L = 0, QB = 1, q0 = 0, rows = 0, qbuf = 1;

  for (long long ub = u0; ub < u1; ub += 2) {
#pragma unroll
    for (int set = 0; set < 2; ++set) {
      const long long u = ub + set;
      {
        // the second unit of the last pair of units may lie past the range: it issues
        // its (empty) loads like every other, so the loads in flight are the same on
        // every path and the compiler's waits stay exact, but computes nothing
        const bool live = u < u1;
        const int b = C.b, ph = C.ph, j = C.j, nb = C.nb;
        const bool seg_first = live && ((u == u0) || (j == 0));
        const bool seg_last = live && ((u == u1 - 1) || (j == nb - 1));
        const int qb = ph % a.qblocks;
        if (seg_first) {
          L = __builtin_amdgcn_readfirstlane(len[b]);
          q0 = qb * a.QB;
          QB = min(a.QB, a.T - q0);
          rows = a.n_rep * QB;
          qpos_s0 = L - a.T + q0 + l16 % QB;
          qpos_s1 = L - a.T + q0 + (16 + l16) % QB;
#pragma unroll
          for (int r = 0; r < 16; ++r) O[r] = 0.f;
          m_s[0] = m_s[1] = -INFINITY;
          l_s[0] = l_s[1] = 0.f;
          m_o = -INFINITY;
          // this pair's Q into the other buffer (its last reader was two pairs ago)
          qbuf ^= 1;
#pragma unroll
          for (int it = 0; it < 2; ++it) {
            const int c = it * AT_THREADS + tid;
            *reinterpret_cast<u32x4_t*>(q_lds + qbuf * (AT_ROWS * AT_KROW) + (c >> 5) * AT_KROW + (c & 31) * 16) =
                qr[it];
          }
        }
        const int key0 = j * AT_BLOCK;

        // 1. stage V, then Q of unit u + 1 and V of unit u + 2 into the registers just freed
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = i * AT_THREADS + tid;
          *reinterpret_cast<u32x4_t*>(v_lds + (c >> 5) * AT_KROW + (c & 31) * 16) = vr[set][i];
        }
        const bool live2 = u + 2 < u1;
        issue_q(X1, u + 1 < u1 && X1.j == 0);
        issue_v(set, X2, live2);
        lds_barrier();

        // 2. S^T for keys [16 w, 16 w + 16) x rows [0, 32): K from registers, Q^T from LDS
        f32x4 S[2];
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) S[r2][jj] = 0.f;
        if (live) {
          const unsigned char* qrow = q_lds + qbuf * (AT_ROWS * AT_KROW) + l16 * AT_KROW + 16 * g4;
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            const bf16x8 kA = __builtin_bit_cast(bf16x8, kr[set][s]);
            const bf16x8 q0B = *reinterpret_cast<const bf16x8*>(qrow + 64 * s);
            const bf16x8 q1B = *reinterpret_cast<const bf16x8*>(qrow + 16 * AT_KROW + 64 * s);
            S[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, q0B, S[0], 0, 0, 0);
            S[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, q1B, S[1], 0, 0, 0);
          }
        }
        // the K loads of unit u + 2 into the registers S just consumed
        issue_k(set, X2, live2);

        if (live) {
          // 3. mask (key < L and <= the row's query position); this wave's row maxima to
          //    LDS, and P^T against the reference max m_s (the running max as of the last
          //    rescale, the same in every wave), written before the one barrier
          float mx[2], ps[2];
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
            const int row = 16 * r2 + l16;
            const float base = m_s[r2] == -INFINITY ? 0.f : m_s[r2] * a.cl2;
            float p[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) p[jj] = fast_exp2(__builtin_fmaf(S[r2][jj], a.cl2, -base));
            ps[r2] = (p[0] + p[1]) + (p[2] + p[3]);
            const uint32_t lo = (uint32_t)f32_to_bf16(p[0]) | ((uint32_t)f32_to_bf16(p[1]) << 16);
            const uint32_t hi = (uint32_t)f32_to_bf16(p[2]) | ((uint32_t)f32_to_bf16(p[3]) << 16);
            *reinterpret_cast<uint2*>(p_lds + row * AT_PROW + (16 * wave + 4 * g4) * 2) = make_uint2(lo, hi);
          }
          lds_barrier();
          // 4. the block maxima of all waves.  While no row's maximum exceeds its reference
          //    by more than 16 in the exponent (weights up to 2^16, safe in bf16 P and fp32
          //    sums), P^T stands and nothing is rescaled; otherwise (always at a pair's first
          //    block) every wave moves the references to the running maxima, rescales l and
          //    O, and rewrites its P^T.  Every wave evaluates all 32 rows from the same LDS
          //    maxima and references, so all take the same branch.
          float mb[2];
          bool big = false;
#pragma unroll
          for (int r2 = 0; r2 < 2; ++r2) {
            const int row = 16 * r2 + l16;
            mb[r2] = m_lds[row];
#pragma unroll
            for (int ww = 1; ww < AT_WAVES; ++ww) mb[r2] = fmaxf(mb[r2], m_lds[ww * AT_ROWS + row]);
            big = big || (mb[r2] - m_s[r2]) * a.cl2 > 16.f;   // false when both are -inf
          }
          float mbo = m_lds[l32];
#pragma unroll
          for (int ww = 1; ww < AT_WAVES; ++ww) mbo = fmaxf(mbo, m_lds[ww * AT_ROWS + l32]);
          big = big || (mbo - m_o) * a.cl2 > 16.f;
          if (__builtin_amdgcn_readfirstlane((int)(__ballot(big) != 0))) {
#pragma unroll
            for (int r2 = 0; r2 < 2; ++r2) {
              const int row = 16 * r2 + l16;
              const float mn = fmaxf(m_s[r2], mb[r2]);
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
            const float mn = fmaxf(m_o, mbo);
            const float alpha = mn == -INFINITY ? 1.f : fast_exp2((m_o - mn) * a.cl2);
            m_o = mn;
            O *= alpha;
            lds_barrier();
          } else {
            l_s[0] += ps[0];
            l_s[1] += ps[1];
          }
          // 5. O^T[32 w .. 32 w + 32) += V^T P^T over the 128 keys
#pragma unroll
          for (int ks = 0; ks < AT_BLOCK / 16; ++ks) {
            const bf16x8 pB = *reinterpret_cast<const bf16x8*>(p_lds + l32 * AT_PROW + (16 * ks + 8 * h2) * 2);
            const unsigned char* vcol = v_lds + (16 * ks + 8 * h2) * AT_KROW + (32 * wave + l32) * 2;
            bf16x8 vA;
#pragma unroll
            for (int e = 0; e < 8; ++e) vA[e] = *reinterpret_cast<const __bf16*>(vcol + e * AT_KROW);
            O = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vA, pB, O, 0, 0, 0);
          }
          lds_barrier();

          if (seg_last) {
            // thread-derived addresses are recomputed from an opaque copy of the thread
            // index here, not hoisted out of the unit loop (where they would not fit the
            // registers next to the two K/V units in flight)
            int t = tid;
            asm volatile("" : "+v"(t));
            const int tl = t & 63, tw = t >> 6, t32 = tl & 31, th2 = tl >> 5;
            // ---- row sums: lanes sharing a row, then waves ----
#pragma unroll
            for (int r2 = 0; r2 < 2; ++r2) {
              float l = l_s[r2];
              l += __shfl_xor(l, 16, 64);
              l += __shfl_xor(l, 32, 64);
              if (tl < 16) l_lds[tw * AT_ROWS + 16 * r2 + tl] = l;
            }
            // O^T -> LDS as O[row][d] (the V block region is free until the next staging)
            float* o_lds = reinterpret_cast<float*>(v_lds);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int d = 32 * tw + 8 * (r >> 2) + 4 * th2 + (r & 3);
              o_lds[t32 * AT_OROW + d] = O[r];
            }
            if (th2 == 0 && tw == 0) m_lds[t32] = m_o;
            lds_barrier();
            const int pair = b * PH + ph;
            // this workgroup's piece of the pair, in slot w + pair (unique: pieces are ordered
            // in both w and pair).  The combine kernel finishes every pair, so no gate load
            // here: waiting on a late load would drain the K/V loads in flight.
            float* part = a.ws + ((size_t)w + pair) * AT_PART;
            if (t < AT_ROWS) {
              float l = 0.f;
#pragma unroll
              for (int ww = 0; ww < AT_WAVES; ++ww) l += l_lds[ww * AT_ROWS + t];
              part[t] = m_lds[t];
              part[AT_ROWS + t] = l;
            }
            for (int c = t; c < rows * (AT_D / 4); c += AT_THREADS) {
              const int r = c / (AT_D / 4), d0 = (c % (AT_D / 4)) * 4;
              const float* src = o_lds + r * AT_OROW + d0;
              *reinterpret_cast<float4*>(part + 2 * AT_ROWS + r * AT_D + d0) =
                  make_float4(src[0], src[1], src[2], src[3]);
            }
            lds_barrier();  // o_lds / l_lds / m_lds read before the next staging overwrites them
          }
        }
        C = X1;
        X1 = X2;
        X2 = advance(X2);
      }
    }
  }
}

// Merge the pieces of pair blockIdx.y for row blockIdx.x and apply the gate: thread d
// owns output column d; piece weights exp(m_s - M) live in LDS.  Every pair is
// finished here (one piece when one workgroup covered it); pairs with no keys get zeros.
// The pieces' workgroup range comes from the table the main kernel wrote.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  __shared__ float wsc[1024];   // piece weights (0 for workgroups with no units)
  __shared__ float lsc[1024];   // piece row sums
  __shared__ float red[8];
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
  const int4 te = reinterpret_cast<const int4*>(a.ws + (size_t)(a.nw + a.B * PH) * AT_PART)[pair];
  const int wf = te.x, wl = te.y;
  const long long U = (long long)(((uint64_t)(uint32_t)te.w << 32) | (uint32_t)te.z);
  if (wf < 0) {   // a pair with no keys
    a.out[o] = 0;
    return;
  }
  // pieces: slot w + pair of every workgroup w in [wf, wl] whose range is not empty
  // (with fewer blocks than workgroups, empty workgroups sit between the owners)
  const int np = wl - wf + 1;
  const float* base = a.ws + ((size_t)wf + pair) * AT_PART;
  // the output column of the first 16 pieces, in flight during the weight reductions
  // (index clamped into the pieces: dead or extra slots are never weighted in)
  const float* col = base + 2 * AT_ROWS + r * AT_D + tid;
  float vv[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) vv[s] = col[(size_t)min(s, np - 1) * AT_PART];
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
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float wgt = s < np ? wsc[s] : 0.f;
    acc += wgt != 0.f ? vv[s] * wgt : 0.f;   // junk in dead slots is never weighted in
  }
#pragma unroll 8
  for (int s = 16; s < np; ++s) {
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

// Workspace: one fp32 piece per workgroup plus one per pair, then the combine's table
// (one int4 per pair).
static long long attn_ws_bytes(long long nw, long long pairs) {
  return (nw + pairs) * AT_PART * (long long)sizeof(float) + pairs * 16;
}

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

// Workgroups of the balanced grid: `grid` if positive, else one per CU of the current
// device.  A piece count per pair above the combine's table size is refused.
static int attn_grid(int grid) {
  if (grid > 0) return grid;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  return cus > 0 ? cus : -1;
}

LOLLM_API long long lollm_attn_workspace_bytes(int B, int T, int Hq, int Hkv, int D,
                                               int max_len, int grid) {
  int n_rep, QB, qblocks;
  if (attn_geometry(B, T, Hq, Hkv, D, max_len, &n_rep, &QB, &qblocks)) return -1;
  const int nw = attn_grid(grid);
  if (nw <= 0) return -1;
  return attn_ws_bytes(nw, (long long)B * Hkv * qblocks);
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
  const long long need = attn_ws_bytes(nw, (long long)B * Hkv * qblocks);
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
  hipLaunchKernelGGL(attn_verify_kernel, dim3(nw), dim3(AT_THREADS), AT_LDS_BYTES, st, a);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(AT_ROWS, B * Hkv * qblocks), dim3(256), 0, st, a);
  return launch_status();
}

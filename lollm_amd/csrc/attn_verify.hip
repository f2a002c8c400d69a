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
// are dealt out in equal contiguous ranges to a fixed grid of one 4-wave workgroup per
// CU.  Every workgroup therefore streams the same number of bytes whatever the context
// lengths, and no CU idles while another finishes a long sequence.  Each workgroup
// leaves one partial (m, l, O) per pair it touched; a combine kernel merges the pieces
// of every pair and applies the gate.
//
// Inside a workgroup the four waves split every unit by keys (wave w: keys 32 w ..
// 32 w + 31) and run independent online softmaxes over them, so the main loop has no
// barrier and no exchange between waves:
//   - K: each wave loads its 32 keys straight into the S MFMA A operand (registers,
//     one unit ahead: with V two units ahead that keeps a wave's loads in flight under
//     the 63 that vmcnt counts, so issuing a load never stalls the wave);
//   - V: each wave's 32 rows arrive by LDS DMA (buffer_load ... lds, two units ahead)
//     into its own part of the unit's LDS set, and are read back as the A operand of
//     O^T += V^T P^T with the transposing LDS read (ds_read_b64_tr_b16), which hands
//     each lane 4 consecutive keys of one column;
//   - Q: the pair's 32 rows are staged in LDS at the pair's first unit and read as the
//     S MFMA B operand;
//   - S^T (32 keys x 32 rows) and O^T (256 columns x 32 rows) are 32x32x16 MFMAs; the
//     S^T accumulator already holds P^T in the order the O^T MFMA consumes it, so P
//     never leaves registers;
//   - the running max of a row only moves (and l, O are rescaled) when a block's
//     maximum exceeds it by more than 16 in the exponent.
// At the end of a pair the four waves' (m, l, O) are merged through the free LDS set
// into the workgroup's piece.
#include "common.h"

namespace lollm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int AT_D = 256;            // head dim
constexpr int AT_ROWS = 32;          // MFMA rows per pair (n_rep x QB)
constexpr int AT_BLOCK = 128;        // keys per block
constexpr int AT_MAXB = 512;         // sequences per call (prefix table in LDS)
constexpr int AT_PART = 2 * AT_ROWS + AT_ROWS * AT_D;  // floats per partial

struct AttnArgs {
  const uint16_t* q;       // (B, T, Hq, D)
  const uint16_t* kc;      // K cache
  const uint16_t* vc;      // V cache
  const int32_t* kv_len;   // (B) keys per sequence, the T new ones included
  const uint16_t* gate;    // (B, T, Hq * D) or null
  uint16_t* out;           // (B, T, Hq * D)
  float* ws;               // partials: (nw + pairs) x AT_PART, then the combine table
  long long seq_stride, head_stride;  // cache strides in elements
  int B, T, Hq, Hkv, n_rep, QB, qblocks, max_len, nw;
  float cl2;               // scale * log2(e)
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

__device__ __forceinline__ int seq_len(const AttnArgs& a, int b) {
  return min(max(a.kv_len[b], 0), a.max_len);  // never past the cache capacity
}

__device__ __forceinline__ int nblk_of(int L) { return (L + AT_BLOCK - 1) / AT_BLOCK; }

// First unit of workgroup w and the workgroup that owns unit u, for U units dealt
// out to nw workgroups in equal contiguous ranges: w owns [U w / nw, U (w+1) / nw).
__device__ __forceinline__ long long unit_begin(long long U, int w, int nw) {
  return U * w / nw;
}
__device__ __forceinline__ int unit_owner(long long U, long long u, int nw) {
  return (int)(((u + 1) * nw - 1) / U);
}

// Buffer loads through a descriptor over [base, base + bytes): offsets past the end read
// zeros without touching memory.  AUX = 2 is the non-temporal hint.
template <int AUX>
__device__ __forceinline__ u32x4_t at_bload(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, AUX));
}

// Position of a unit in the pair-major block order: sequence b, pair ph of it, block j
// of the pair's nb blocks.
struct AtCursor {
  int b, ph, j, nb;
};

constexpr int AW_WAVES = 4;
constexpr int AW_THREADS = 64 * AW_WAVES;
constexpr int AW_WKEYS = AT_BLOCK / AW_WAVES;        // 32 keys of each block per wave
constexpr int AW_VPAIR = 2 * AT_D * 2 + 64;          // two V rows (one DMA) + 64 bytes of padding
constexpr int AW_VWAVE = AW_WKEYS / 2 * AW_VPAIR;     // 17 KB: one wave's V rows of a block
constexpr int AW_VSET = AW_WAVES * AW_VWAVE;          // the V rows of one block
constexpr int AW_QROW = AT_D * 2 + 16;                // padded Q row in LDS
constexpr int AW_OROW = AT_D / 2 + 4;                 // padded floats per row of an O half-dump
static_assert(AW_WAVES * AT_ROWS * AW_OROW * 4 <= AW_VSET, "the O dump fits a V set");
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// pre[b] = blocks of sequences 0..b-1 (pre[0] = 0), for b = 0..B, and len[b] = the
// clamped key count of sequence b, built in LDS by the whole workgroup (so the main
// loop never waits on a global load to address the next block).  Returns pre[B].
__device__ int build_prefix(const AttnArgs& a, int* pre, int* len, int* tmp) {
  constexpr int WAVES = AW_WAVES;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int carry = 0;
  if (tid == 0) pre[0] = 0;
  for (int base = 0; base < a.B; base += AW_THREADS) {
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
    for (int w = 0; w < WAVES; ++w) {
      if (w < wave) before += tmp[w];
      all += tmp[w];
    }
    if (b < a.B) pre[b + 1] = before + v;
    carry = all;
    __syncthreads();
  }
  return carry;
}

// Workgroup barrier after this wave's LDS accesses complete; the compiler sees a memory
// clobber (no LDS access moves across it) but no fence, so global loads and LDS DMA in
// flight are not drained.
__device__ __forceinline__ void aw_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__global__ __launch_bounds__(AW_THREADS, 1) void attn_verify_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char vs0[AW_VSET];   // V of even units
  __shared__ __attribute__((aligned(16))) unsigned char vs1[AW_VSET];   // V of odd units
  __shared__ __attribute__((aligned(16))) unsigned char qs[AT_ROWS * AW_QROW];   // Q of the pair
  __shared__ float mx[AW_WAVES][32], lx[AW_WAVES][32];
  __shared__ int pre[AT_MAXB + 1], len[AT_MAXB], tmp[AW_WAVES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int w = blockIdx.x;
  const int PH = a.Hkv * a.qblocks;

  const long long U = (long long)PH * build_prefix(a, pre, len, tmp);
  {
    const int npairs = a.B * PH;
    int4* tab = reinterpret_cast<int4*>(a.ws + (size_t)(a.nw + npairs) * AT_PART);
    for (int p = w * AW_THREADS + tid; p < npairs; p += a.nw * AW_THREADS) {
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

  // zero both V sets once: rows past a sequence's end are never loaded, and what they
  // hold must stay finite (their P is 0)
  for (int i = tid; i < AW_VSET / 16; i += AW_THREADS) {
    *reinterpret_cast<uint4*>(vs0 + 16 * i) = make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4*>(vs1 + 16 * i) = make_uint4(0, 0, 0, 0);
  }
  __syncthreads();

  // Loads of a unit (all unconditional; a unit past the range gets an empty descriptor).
  //   K: wave w's 32 keys straight into the S MFMA A operand (lane: key 32 w + l32,
  //      16 bytes at d chunk 2 ks + h for k-step ks), one unit ahead
  //   V: wave w's 32 rows by LDS DMA into its part of the unit's set, 2 rows (1 KB)
  //      per instruction, 64 bytes of padding after each pair of rows (so that the
  //      transposing reads of 8 consecutive rows hit every bank at most twice)
  //   Q: the next pair's 32 rows into registers one unit ahead (thread t: row t / 32 + 8 i,
  //      chunk t % 32), staged in LDS (padded rows) at the pair's first unit and read as
  //      the S MFMA B operand (lane: row l32, d chunk 2 ks + h)
  u32x4_t kr[16], qr[4];
  auto rsrc_of = [&](const uint16_t* cache, const AtCursor& X, bool live) {
    const int kvh = live ? X.ph / a.qblocks : 0;
    const uint32_t bytes = live ? (uint32_t)__builtin_amdgcn_readfirstlane(len[X.b]) * (AT_D * 2) : 0u;
    const uint16_t* base = cache + (live ? (size_t)X.b * a.seq_stride + (size_t)kvh * a.head_stride : 0);
    return buf_rsrc(base, bytes);
  };
  auto issue_k = [&](const AtCursor& X, bool live) {
    const __amdgpu_buffer_rsrc_t rs = rsrc_of(a.kc, X, live);
    const uint32_t ko = (uint32_t)(X.j * AT_BLOCK + AW_WKEYS * wave + l32) * (AT_D * 2) + 16u * h;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) kr[ks] = at_bload<0>(rs, ko + 32u * ks, 0u);
  };
  auto issue_v = [&](unsigned char* vset, const AtCursor& X, bool live) {
    const __amdgpu_buffer_rsrc_t rs = rsrc_of(a.vc, X, live);
    unsigned char* dst = vset + wave * AW_VWAVE;
    const uint32_t vo = (uint32_t)(X.j * AT_BLOCK + AW_WKEYS * wave) * (AT_D * 2) + 16u * lane;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + AW_VPAIR * i), 16, vo, 1024u * i, 0, 2);
  };
  auto issue_q = [&](const AtCursor& X, bool load) {
    const int kvh = load ? X.ph / a.qblocks : 0, qb = load ? X.ph % a.qblocks : 0;
    const int q0_ = qb * a.QB, QB_ = min(a.QB, a.T - q0_), rows_ = a.n_rep * QB_;
    const uint32_t bytes = load ? (uint32_t)a.T * (uint32_t)a.Hq * (AT_D * 2) : 0u;
    const uint16_t* base = a.q + (load ? (size_t)X.b * a.T * a.Hq * AT_D : 0);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(base, bytes);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int r = (tid >> 5) + 8 * ii, c = tid & 31;
      const int hr = r / QB_, i = r % QB_;
      const uint32_t qo = r < rows_ ? ((uint32_t)(q0_ + i) * (uint32_t)a.Hq + (uint32_t)(kvh * a.n_rep + hr)) *
                                          (AT_D * 2) + 16u * c
                                    : 0x80000000u;
      qr[ii] = at_bload<0>(rs, qo, 0u);
    }
  };

  AtCursor X1 = advance(C), X2 = advance(X1);
  issue_q(C, true);
  issue_k(C, true);
  issue_v(vs0, C, true);
  issue_v(vs1, X1, u0 + 1 < u1);

  f32x16 O[8];            // O^T: d-tile dt (32 columns) x the 32 rows; lane row = l32
  float m_ref = -INFINITY, l_s = 0.f;
  int qpos = 0, L = 0;

  for (long long ub = u0; ub < u1; ub += 2) {
#pragma unroll
    for (int set = 0; set < 2; ++set) {
      unsigned char* vset = set ? vs1 : vs0;
      const long long u = ub + set;
      const bool live = u < u1;
      const int b = C.b, ph = C.ph, j = C.j, nb = C.nb;
      const bool seg_first = live && ((u == u0) || (j == 0));
      const bool seg_last = live && ((u == u1 - 1) || (j == nb - 1));
      if (seg_first) {
        const int qb = ph % a.qblocks;
        L = __builtin_amdgcn_readfirstlane(len[b]);
        const int q0 = qb * a.QB, QB = min(a.QB, a.T - q0);
        qpos = L - a.T + q0 + l32 % QB;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) O[dt][r] = 0.f;
        m_ref = -INFINITY;
        l_s = 0.f;
        // (the previous pair's last unit ended with barriers: no wave still reads qs)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          *reinterpret_cast<u32x4_t*>(qs + ((tid >> 5) + 8 * ii) * AW_QROW + 16 * (tid & 31)) = qr[ii];
        aw_barrier();
      }
      const bool live2 = u + 2 < u1;
      // Q of the next unit's pair (staged at that unit's start)
      issue_q(X1, u + 1 < u1 && (X1.j == 0));

      // S^T (32 keys x 32 rows) = K Q^T
      f32x16 S;
#pragma unroll
      for (int r = 0; r < 16; ++r) S[r] = 0.f;
      if (live) {
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
          const bf16x8 qb = *reinterpret_cast<const bf16x8*>(qs + l32 * AW_QROW + 16 * h + 32 * ks);
          S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[ks]), qb, S, 0, 0, 0);
        }
      }
      issue_k(X1, u + 1 < u1);   // K of the next unit into the registers S consumed

      if (live) {
        // mask: acc r holds key 32 wave + 8 (r / 4) + 4 h + r % 4 of the block
        const int kb = j * AT_BLOCK + AW_WKEYS * wave + 4 * h;
        const int lim = min(L - 1, qpos) - kb;
        float bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 8 * (r >> 2) + (r & 3);
          S[r] = kk <= lim ? S[r] : -INFINITY;
          bm = fmaxf(bm, S[r]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        // the reference max moves (and l, O are rescaled) only when a row's block max
        // exceeds it by more than 16 in the exponent (always at a pair's first block).
        // The decision is the row's own (the ballot only skips the rescale when no row
        // needs one; other rows scale by exactly 1), so a row's bits do not depend on
        // which other rows share the pair -- the verify length T, the padding rows.
        const bool big = (bm - m_ref) * a.cl2 > 16.f;
        if (__builtin_amdgcn_readfirstlane((int)(__ballot(big) != 0))) {
          const float mn = big ? fmaxf(m_ref, bm) : m_ref;
          const float alpha = (!big || mn == -INFINITY) ? 1.f : fast_exp2((m_ref - mn) * a.cl2);
          m_ref = mn;
          l_s *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) O[dt] *= alpha;
        }
        const float base = m_ref == -INFINITY ? 0.f : m_ref * a.cl2;
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = fast_exp2(__builtin_fmaf(S[r], a.cl2, -base));
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) ps += p[r];
        l_s += ps;
        bf16x8 P[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          u32x4_t pw;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pw[e] = (uint32_t)f32_to_bf16(p[8 * k2 + 2 * e]) | ((uint32_t)f32_to_bf16(p[8 * k2 + 2 * e + 1]) << 16);
          P[k2] = __builtin_bit_cast(bf16x8, pw);
        }

        // O^T += V^T P^T: A = V^T from LDS by transposing reads (lane: column 32 dt + l32,
        // keys 16 ks + 4 h + 0..3 and 16 ks + 8 + 4 h + 0..3, the order P holds them in)
        // lane's rows 16 ks + 8 q + x (x = 4 h + (lane % 16) / 4), columns 32 dt +
        // 16 ((lane / 16) % 2) + 4 (lane % 4): a per-lane base plus constant offsets
        const int x = 4 * h + ((lane & 15) >> 2);
        const unsigned char* vw = vset + wave * AW_VWAVE + (x >> 1) * AW_VPAIR + (x & 1) * (AT_D * 2) +
                                  32 * ((lane >> 4) & 1) + 8 * (lane & 3);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_t*)(vw + 8 * ks * AW_VPAIR + 64 * dt));
            const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_t*)(vw + (8 * ks + 4) * AW_VPAIR + 64 * dt));
            const u32x2_t w0 = __builtin_bit_cast(u32x2_t, v0), w1 = __builtin_bit_cast(u32x2_t, v1);
            const u32x4_t wa = {w0.x, w0.y, w1.x, w1.y};
            const bf16x8 vA = __builtin_bit_cast(bf16x8, wa);
            O[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vA, P[ks], O[dt], 0, 0, 0);
          }
        }
      }

      if (seg_last) {
        // merge the four waves' (m, l, O) of this pair into the workgroup's piece, in two
        // halves of d through the free V set: each wave dumps its O (straight from the
        // accumulators), then every thread sums one row's 16 columns with the waves'
        // weights exp(m_w - M)
        const float lrow = l_s + __shfl_xor(l_s, 32, 64);
        aw_barrier();   // every wave is done reading this set
        if (h == 0) {
          mx[wave][l32] = m_ref;
          lx[wave][l32] = lrow;
        }
        const int pair = b * PH + ph;
        float* part = a.ws + ((size_t)w + pair) * AT_PART;
        float* dump = reinterpret_cast<float*>(vset);
        const int srow = tid >> 3, sc8 = tid & 7;
        float wgt[AW_WAVES];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              *reinterpret_cast<float4*>(dump + (wave * AT_ROWS + l32) * AW_OROW + 32 * dt + 8 * q + 4 * h) =
                  make_float4(O[4 * half + dt][4 * q], O[4 * half + dt][4 * q + 1], O[4 * half + dt][4 * q + 2],
                              O[4 * half + dt][4 * q + 3]);
          aw_barrier();
          if (half == 0) {
            float M = mx[0][srow];
#pragma unroll
            for (int ww = 1; ww < AW_WAVES; ++ww) M = fmaxf(M, mx[ww][srow]);
            float Lsum = 0.f;
#pragma unroll
            for (int ww = 0; ww < AW_WAVES; ++ww) {
              const float mw = mx[ww][srow];
              wgt[ww] = mw == -INFINITY ? 0.f : fast_exp2((mw - M) * a.cl2);
              Lsum += lx[ww][srow] * wgt[ww];
            }
            if (sc8 == 0) {
              part[srow] = M;
              part[AT_ROWS + srow] = Lsum;
            }
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int ww = 0; ww < AW_WAVES; ++ww) {
              const float4 v = *reinterpret_cast<const float4*>(dump + (ww * AT_ROWS + srow) * AW_OROW + 16 * sc8 + 4 * k);
              acc.x += wgt[ww] * v.x; acc.y += wgt[ww] * v.y; acc.z += wgt[ww] * v.z; acc.w += wgt[ww] * v.w;
            }
            *reinterpret_cast<float4*>(part + 2 * AT_ROWS + srow * AT_D + 128 * half + 16 * sc8 + 4 * k) = acc;
          }
          aw_barrier();   // the dump is read before it is overwritten (and the set refilled)
        }
      }
      // V of unit u + 2 into this set
      issue_v(vset, X2, live2);
      C = X1;
      X1 = X2;
      X2 = advance(X2);
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
  hipLaunchKernelGGL(attn_verify_kernel, dim3(nw), dim3(AW_THREADS), 0, st, a);
  if ((rc = launch_status())) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(AT_ROWS, B * Hkv * qblocks), dim3(256), 0, st, a);
  return launch_status();
}

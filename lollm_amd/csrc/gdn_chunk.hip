// Chunked Gated DeltaNet mixer for long calls (prefill), gfx950.  The layer is the one
// lollm_gdn_layer computes -- causal conv + SiLU (src/qwen3_5/blocks.py:268-286), beta /
// g gating (:313-314), L2 norm of q and k (:124-127), the delta rule, the gated
// RMSNorm (:38-51,324) -- with the delta rule in its parallel
// chunked form (torch_chunk_gated_delta_rule, blocks.py:59-113, which the reference
// runs for every T > 1 call, :316-322), and the same conv-window / state placement as
// the long-call path of gdn_layer.hip (starts from the committed state that the long-call
// prologue wrote to the state half being written, leaves the final state there and the
// final K-1 raw inputs in rows 0 .. K-2 of the window half being written).
//
// One 256-thread workgroup per (sequence b, v-head h) walks the chunks of 64 tokens in
// order.  Per chunk, with gc = cumsum(g) and s = Dk^-0.5:
//   A  = -(beta_i k_i.k_j) exp(gc_i - gc_j), j < i          (:99-100)
//   Tm = (I - A)^-1                                          (:101-103)
//   W  = Tm diag(beta e^gc) K,   V' = Tm diag(beta) V - W S   (:104-105, :113)
//   O  = diag(s e^gc) Q S + [s (q_i.k_j) exp(gc_i - gc_j)]_{j<=i} V'   (:112-115)
//   S <- e^gc_63 S + K^T diag(e^(gc_63 - gc)) V'              (:116-117)
//
// Work split.  The 128 x 128 fp32 state S[key][value] lives in registers: wave w owns
// the value columns 32w .. 32w+31 in the 16x16 MFMA accumulator layout (lane (g, r)
// holds S[16kb + 4g + j][32w + 16u + r]), so V', O and the state update of those
// columns never leave the wave.  The value-independent matrices (k, k^T, q, v^T, Tm
// scaled two ways, W, the masked q.k decay) are shared through LDS.
//
// Arithmetic.  Products run on the bf16 MFMA (16x16x32).  q, k, v are bf16 conv
// outputs and enter exactly; an fp32 operand x enters as hi + lo with hi = bf16(x),
// lo = bf16(x - hi) (16 significant bits), and a product of two fp32 operands takes
// hi.hi + hi.lo + lo.hi, so every product carries a relative error near 2^-17 against
// the reference's fp32 arithmetic, accumulated in fp32.  A product whose B operand
// comes from registers (S, V') contracts in the accumulator's row order: its k slots
// 8g .. 8g+7 hold rows 32s + 4g .. +3 and 32s + 16 + 4g .. +3, and the A operand is
// read from LDS in that same order (two 8-byte reads).
//
// Tm is solved blockwise in fp32: the four 16 x 16 diagonal blocks by the reference's
// row recurrence (one lane per column), the off-diagonal blocks by
// T_ij = T_ii sum_{k=j}^{i-1} A_ik T_kj with fp32 MFMA (16x16x4), while the other three
// waves form the masked q.k decay.
//
// q and k enter the products as their bf16 conv outputs with the L2-norm factors
// rq_t, rk_t applied as fp32 scales (the normalised vectors are never rounded), which
// is the arithmetic of the recurrent kernels, so a prefill and the decode steps after
// it agree.  Tokens past T in the last chunk enter with q = k = v = 0 and
// beta = g = 0 and change nothing, as the reference's zero padding (:77-80).
#include "gdn_common.h"

namespace lollm {

constexpr int GC_C = 64;     // tokens per chunk
constexpr int GC_PW = 136;   // bf16 pitch of 128-wide rows
constexpr int GC_PN = 72;    // bf16 pitch of 64-wide rows
constexpr int GC_PF = 68;    // fp32 pitch of 64-wide rows
constexpr int GC_PO = 132;   // fp32 pitch of the output rows

typedef float gc_f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 gc_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 gc_bf16x2 __attribute__((ext_vector_type(2)));

struct GcSmem {
  union {
    uint16_t kc[GC_C][GC_PW];           // k [t][channel] (conv -> q.k products)
    uint16_t in[2][GC_C][GC_PN];        // hi, lo of the masked s q.k decay [i][j]
  } r1;
  uint16_t kt[GL_DK][GC_PN];            // k^T [channel][t]
  uint16_t qc[GC_C][GC_PW];             // q [t][channel]
  uint16_t vt[GL_DK][GC_PN];            // v^T [channel][t]
  union {
    struct {
      float am[GC_C][GC_PF];            // A (strictly lower)
      float tf[GC_C][GC_PF];            // Tm, lower blocks
    } s;
    uint16_t w[2][GC_C][GC_PW];         // hi, lo of -W [t][key]
  } r2;
  union {
    uint16_t tm[4][GC_C][GC_PN];        // hi, lo of Tm diag(rk beta e^gc), of Tm diag(beta)
    float o[GC_C][GC_PO];               // O (fp32) for the gated norm
  } r3;
  float gcv[GC_C], egv[GC_C], btv[GC_C], rqv[GC_C], rkv[GC_C];
  float fwv[GC_C], f7v[GC_C];  // rk beta e^gc (W), rk e^(gc_63 - gc) (state update)
  uint16_t cw[GL_CH][4];       // conv weights of the head's q, k, v channels
};
static_assert(sizeof(GcSmem) <= 160 * 1024, "LDS budget");

__device__ __forceinline__ float gc_bf(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

__device__ __forceinline__ gc_f32x4 gc_mma(gc_bf16x8 a, gc_bf16x8 b, gc_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ gc_f32x4 gc_mma4(float a, float b, gc_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ gc_bf16x8 gc_ld8(const uint16_t* p) {
  return __builtin_bit_cast(gc_bf16x8, *reinterpret_cast<const u32x4_t*>(p));
}

// k slots 0..3 from p0, 4..7 from p1 (the accumulator row order)
__device__ __forceinline__ gc_bf16x8 gc_ld44(const uint16_t* p0, const uint16_t* p1) {
  const uint2 x = *reinterpret_cast<const uint2*>(p0), y = *reinterpret_cast<const uint2*>(p1);
  return __builtin_bit_cast(gc_bf16x8, u32x4_t{x.x, x.y, y.x, y.y});
}

// hi/lo bf16 of the 8 values p[0..3], q[0..3]
__device__ __forceinline__ void gc_split(gc_f32x4 p, gc_f32x4 q, gc_bf16x8& hi, gc_bf16x8& lo) {
  gc_bf16x8 h, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const __bf16 a = (__bf16)p[j], c = (__bf16)q[j];
    h[j] = a;
    h[j + 4] = c;
    l[j] = (__bf16)(p[j] - (float)a);
    l[j + 4] = (__bf16)(q[j] - (float)c);
  }
  hi = h;
  lo = l;
}

__device__ __forceinline__ uint16_t gc_bits(__bf16 x) { return __builtin_bit_cast(uint16_t, x); }

__device__ __forceinline__ float gc_rbf(float x) { return (float)(__bf16)x; }   // round to bf16

// 16-lane row sum in every lane of the row (DPP: quad xor 1, xor 2, half-row and row
// mirrors)
template <int CTRL> __device__ __forceinline__ float gc_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float gc_row16_sum(float v) {
  v += gc_dpp<0xB1>(v);
  v += gc_dpp<0x4E>(v);
  v += gc_dpp<0x141>(v);
  v += gc_dpp<0x140>(v);
  return v;
}

__device__ __forceinline__ uint32_t gc_pack(float lo, float hi) {
  return (uint32_t)gc_bits((__bf16)lo) | ((uint32_t)gc_bits((__bf16)hi) << 16);
}

// projection column of local channel lc (0..127 q, 128..255 k, 256..383 v) of head h
__device__ __forceinline__ int gc_chan(const GdnLayerArgs& a, int hk, int h, int lc) {
  return lc < GL_DK ? hk * GL_DK + lc
                    : (lc < 2 * GL_DK ? a.key_dim + hk * GL_DK + (lc - GL_DK)
                                      : 2 * a.key_dim + h * GL_DK + (lc - 2 * GL_DK));
}

// Conv work of a chunk: item n of thread tid = (8-channel vector cv of the 48, 4-token
// group tq of the 16) with it = tid + 256 n; its 7 input rows (3 history + 4) are
// loaded ahead of use.  Chunks after the first read the projection through a buffer
// descriptor over this sequence's rows: a row past the call reads as zero (it only
// feeds outputs of tokens past the call), no address is clamped, and a load costs one
// 32-bit add.  The loads are issued unconditionally and nothing touches the loaded
// values before their use, so no wait is placed at the loads and a later wait never
// drains loads issued after these.
constexpr int GC_ITEMS = 3;

__device__ __forceinline__ u32x4_t gc_bload(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}

// The NB blocks T_(j+d, j), d = 4 - NB, of Tm's block diagonal d (64 x 64, 16 x 16 blocks).
template <int NB>
__device__ __forceinline__ void gc_off_diagonal(float (*am)[GC_PF], float (*tf)[GC_PF], int r16, int g4) {
  constexpr int d = 4 - NB;
  gc_f32x4 p[NB], t[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    p[n] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
    t[n] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int kb = 0; kb < d; ++kb)
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int n = 0; n < NB; ++n)
        p[n] = gc_mma4(am[16 * (n + d) + r16][16 * (n + kb) + 4 * s + g4],
                       tf[16 * (n + kb) + 4 * s + g4][16 * n + r16], p[n]);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int n = 0; n < NB; ++n)
      t[n] = gc_mma4(tf[16 * (n + d) + r16][16 * (n + d) + 4 * g4 + s], p[n][s], t[n]);
#pragma unroll
  for (int n = 0; n < NB; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) tf[16 * (n + d) + 4 * g4 + j][16 * n + r16] = t[n][j];
}

__global__ __launch_bounds__(256) void gdn_chunk_kernel(GdnLayerArgs a) {
  __shared__ GcSmem sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;   // MFMA lane coordinates
  const int b = blockIdx.x / a.Hv, h = blockIdx.x % a.Hv;
  const int vpk = a.Hv / a.Hk, hk = h / vpk;
  const bool write_qk = (h % vpk) == 0;
  const int Km1 = a.K - 1;   // == 3 on this path
  constexpr size_t SS = (size_t)GL_DK * GL_DK;
  int off = a.conv_off[b];
  off = off < 0 ? 0 : (off > 2 * a.W - Km1 ? 2 * a.W - Km1 : off);
  const int wbase = off >= a.W ? 0 : a.W;
  // the state half written by this call: it already holds the committed state (the
  // long-call prologue rebuilt it there) and receives the final state
  float* st_io = a.rec + ((size_t)(b * 2 + ((a.rec_half[b] & 1) ^ 1)) * a.Hv + h) * SS;
  const size_t win_b = (size_t)b * 2 * a.W;
  const float qscale = rsqrtf((float)GL_DK);
  const float a_log = a.A_log[h], dtb = a.dt_bias[h];
  const int vcol = 32 * wave;   // first value column of this wave


  // ---- initial state: this wave's 32 value columns, accumulator layout ----
  gc_f32x4 st[8][2];
  {
    const float* s0 = st_io;
    const float keep = a.fresh ? 0.f : 1.f;   // a fresh sequence starts from S = 0
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          st[kb][u][j] = keep * s0[(size_t)(16 * kb + 4 * g4 + j) * GL_DK + vcol + 16 * u + r16];
  }

  int c0n[GC_ITEMS];   // projection column of each conv item's first channel
#pragma unroll
  for (int n = 0; n < GC_ITEMS; ++n) c0n[n] = gc_chan(a, hk, h, 8 * ((tid + 256 * n) % 48));
  const uint16_t* projb = a.proj + (size_t)b * a.T * a.P;   // this sequence's projection rows
  const uint32_t P2 = (uint32_t)a.P * 2u;                    // bytes per projection row
  // (base and size made explicitly uniform, so the descriptor stays in scalar registers)
  const uint64_t pbase = (uint64_t)projb;
  const uint32_t plo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)pbase);
  const uint32_t phi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(pbase >> 32));
  const uint64_t pbu = ((uint64_t)phi << 32) | (uint64_t)plo;   // no sign extension of the low word
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pbu, (short)0, __builtin_amdgcn_readfirstlane((int)((uint32_t)a.T * P2)), 0x00020000);
  // byte offsets, relative to the chunk's first row: item n's first input row (3 before
  // its group), the gating b of token tid & 63, z of norm row tid / 16
  uint32_t roff[GC_ITEMS];
#pragma unroll
  for (int n = 0; n < GC_ITEMS; ++n)
    roff[n] = (uint32_t)((4 * ((tid + 256 * n) / 48) - 3) * (int)P2 + 2 * c0n[n]);
  const uint32_t boff = (uint32_t)(tid & (GC_C - 1)) * P2 + 2u * (uint32_t)(a.C + a.value_dim + h);
  const uint32_t zoff = (uint32_t)(tid >> 4) * P2 + 2u * (uint32_t)(a.C + h * GL_DK + (tid & 15) * 8);
  u32x4_t raw[GC_ITEMS][7];
  uint16_t braw, araw;
  // the first chunk's history rows come from the committed conv window
#pragma unroll
  for (int n = 0; n < GC_ITEMS; ++n) {
    const int t4 = 4 * ((tid + 256 * n) / 48);
#pragma unroll
    for (int r = 0; r < 7; ++r) {
      const int t = t4 - 3 + r;
      const uint16_t* src = t < 0 ? a.win + (win_b + off + 3 + t) * a.C + c0n[n]
                                  : projb + (size_t)(t < a.T ? t : a.T - 1) * a.P + c0n[n];
      raw[n][r] = *reinterpret_cast<const u32x4_t*>(src);
    }
  }
  braw = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(prs, boff, 0, 0);
  araw = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(prs, boff + 2u * a.Hv, 0, 0);
  float nwf[8];   // gated-norm weight of this thread's 8 columns
  {
    const uint4 nw = *reinterpret_cast<const uint4*>(a.norm_w + (tid & 15) * 8);
    const uint32_t nd[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) nwf[e] = __uint_as_float(e & 1 ? nd[e >> 1] & 0xffff0000u : nd[e >> 1] << 16);
  }
  if (tid < GL_CH / 2)   // two channels (16 bytes) per thread
    *reinterpret_cast<u32x4_t*>(&sh.cw[2 * tid][0]) =
        *reinterpret_cast<const u32x4_t*>(a.conv_w + (size_t)gc_chan(a, hk, h, 2 * tid) * 4);
  __syncthreads();

  for (int t0 = 0; t0 < a.T; t0 += GC_C) {
    // lane coordinates re-derived per chunk from an opaque copy of the thread index, so
    // the compiler recomputes LDS addresses in the loop instead of holding (and
    // spilling) every one of them across it
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, r16 = lane & 15, g4 = lane >> 4;
    // ================= conv + SiLU, L2-norm factors; beta, g, cumsum(g) =================
    // (every reader of the chunk buffers passed the barrier before the previous norm)
#pragma unroll
    for (int n = 0; n < GC_ITEMS; ++n) {
      const int it = tid + 256 * n, cv = it % 48, tq = it / 48;
      const int nvalid = a.T - (t0 + 4 * tq);   // tokens of the group inside the call
      // the 4-tap conv as two bf16 dot products per output: weights (tap 0, 1) and
      // (tap 2, 3) of a channel are consecutive bf16 pairs; the inputs are paired
      // (row r, row r + 1) per channel with a byte permute
      const u32x4_t* cwp = reinterpret_cast<const u32x4_t*>(&sh.cw[8 * cv][0]);
      uint32_t w01[8], w23[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4_t cw = cwp[q];
        w01[2 * q] = cw[0]; w23[2 * q] = cw[1]; w01[2 * q + 1] = cw[2]; w23[2 * q + 1] = cw[3];
      }
      uint32_t prs[6][8];   // (row r, row r + 1) of channel e
#pragma unroll
      for (int r = 0; r < 6; ++r)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          prs[r][2 * p] = __builtin_amdgcn_perm(raw[n][r + 1][p], raw[n][r][p], 0x05040100u);
          prs[r][2 * p + 1] = __builtin_amdgcn_perm(raw[n][r + 1][p], raw[n][r][p], 0x07060302u);
        }
      uint32_t pk[4][4];   // token r: bf16 pairs (channels 2p, 2p + 1)
      float ssq[4];        // token r: sum of squares over the 8 channels
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ssq[r] = 0.f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          float o2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int ee = 2 * p + u;
            float acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gc_bf16x2, prs[r][ee]),
                                                        __builtin_bit_cast(gc_bf16x2, w01[ee]), 0.f, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gc_bf16x2, prs[r + 2][ee]),
                                                  __builtin_bit_cast(gc_bf16x2, w23[ee]), acc, false);
            o2[u] = silu_g(gc_rbf(acc));
          }
          const uint32_t pv = gc_pack(o2[0], o2[1]);
          pk[r][p] = r < nvalid ? pv : 0u;
          // the two squares in one bf16 dot product (exact products, fp32 sum)
          ssq[r] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gc_bf16x2, pk[r][p]),
                                                   __builtin_bit_cast(gc_bf16x2, pk[r][p]), ssq[r], false);
        }
      }
      // the 16 lanes of a DPP row hold the 16 channel vectors of one kind (q, k or v)
      // for the same 4 tokens: the row sum is the squared norm over 128 channels
#pragma unroll
      for (int r = 0; r < 4; ++r) ssq[r] = gc_row16_sum(ssq[r]);
      const int kind = cv >> 4, col = (cv & 15) * 8;   // 0 q, 1 k, 2 v
      if (kind < 2 && (cv & 15) == 0) {
        float* dstv = kind == 0 ? sh.rqv : sh.rkv;
#pragma unroll
        for (int r = 0; r < 4; ++r) dstv[4 * tq + r] = rsqrtf(ssq[r] + 1e-6f);
      }
      if (kind < 2) {
        uint16_t* dst = kind == 0 ? &sh.qc[0][0] : &sh.r1.kc[0][0];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<u32x4_t*>(dst + (4 * tq + r) * GC_PW + col) =
              u32x4_t{pk[r][0], pk[r][1], pk[r][2], pk[r][3]};
      }
      if (kind > 0) {
        uint16_t* dst = kind == 1 ? &sh.kt[0][0] : &sh.vt[0][0];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          uint32_t c[2];   // channel e of tokens (2 r2, 2 r2 + 1)
#pragma unroll
          for (int r2 = 0; r2 < 2; ++r2)
            c[r2] = __builtin_amdgcn_perm(pk[2 * r2 + 1][e >> 1], pk[2 * r2][e >> 1],
                                          e & 1 ? 0x07060302u : 0x05040100u);
          *reinterpret_cast<uint2*>(dst + (col + e) * GC_PN + 4 * tq) = make_uint2(c[0], c[1]);
        }
      }
    }
    if (wave == 0) {   // lane = token
      float gg = 0.f, bb = 0.f;
      if (t0 + lane < a.T) {
        const float x = gc_bf(araw) + dtb;   // softplus with torch's linear range above 20
        gg = -__expf(a_log) * (x > 20.f ? x : __logf(1.f + __expf(x)));
        bb = gc_rbf(__builtin_amdgcn_rcpf(1.f + __expf(-gc_bf(braw))));
      }
      // cumsum(g) over the chunk as an inclusive lane scan
      float gc = gg;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float up = __shfl_up(gc, d, 64);
        gc += lane >= d ? up : 0.f;
      }
      sh.btv[lane] = bb;
      sh.gcv[lane] = gc;
      sh.egv[lane] = __expf(gc);
    }
    // z of this chunk for the gated norm (rows 16 n + tid / 16, 8 columns), issued after
    // the conv's loads were consumed and in flight until the end of the chunk
    u32x4_t zreg[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) zreg[n] = gc_bload(prs, zoff + (uint32_t)(t0 + 16 * n) * P2);
    __syncthreads();
    if (tid < GC_C) {
      sh.fwv[tid] = sh.rkv[tid] * sh.btv[tid] * sh.egv[tid];
      sh.f7v[tid] = sh.rkv[tid] * __expf(sh.gcv[GC_C - 1] - sh.gcv[tid]);
    }
    // ================= A = -(beta_i k_i.k_j) exp(gc_i - gc_j), j < i =================
    // the 10 lower 16 x 16 tiles (ti >= tj), dealt to the waves
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      const int q = wave + 4 * n;
      if (q < 10) {
        const int ti = q < 1 ? 0 : (q < 3 ? 1 : (q < 6 ? 2 : 3));
        const int tj = q - ti * (ti + 1) / 2;
        gc_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
          acc = gc_mma(gc_ld8(&sh.r1.kc[16 * ti + r16][32 * s + 8 * g4]),
                       gc_ld8(&sh.r1.kc[16 * tj + r16][32 * s + 8 * g4]), acc);
        const int i0 = 16 * ti + 4 * g4, jj = 16 * tj + r16;
        const float4 bt = *reinterpret_cast<const float4*>(&sh.btv[i0]);
        const float4 rk = *reinterpret_cast<const float4*>(&sh.rkv[i0]);
        const float4 gi = *reinterpret_cast<const float4*>(&sh.gcv[i0]);
        const float bta[4] = {bt.x, bt.y, bt.z, bt.w}, rka[4] = {rk.x, rk.y, rk.z, rk.w};
        const float gia[4] = {gi.x, gi.y, gi.z, gi.w};
        const float rkj = sh.rkv[jj], gj = sh.gcv[jj];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sh.r2.s.am[i0 + j][jj] = jj < i0 + j ? -bta[j] * (acc[j] * rka[j] * rkj) * __expf(gia[j] - gj) : 0.f;
      }
    }
    __syncthreads();
    // ======== Tm = (I - A)^-1 (wave 0) | masked s q.k decay (waves 1..3) ========
    gc_f32x4 qk[4];   // this wave's q.k decay tiles, written after the barrier
    if (wave == 0) {
      // diagonal blocks: lane = 16 blk + column; rows broadcast from LDS per block
      {
        const int base = 16 * (lane >> 4), c = lane & 15;
        float col[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) col[m] = sh.r2.s.am[base + m][base + c];
#pragma unroll
        for (int i = 1; i < 16; ++i) {
          float acc = 0.f;
#pragma unroll
          for (int m4 = 0; m4 < i; m4 += 4) {
            const float4 rowv = *reinterpret_cast<const float4*>(&sh.r2.s.am[base + i][base + m4]);
            const float rv[4] = {rowv.x, rowv.y, rowv.z, rowv.w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (m4 + u < i) acc = fmaf(rv[u], col[m4 + u], acc);
          }
          col[i] += acc;
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) sh.r2.s.tf[base + m][base + c] = col[m] + (m == c ? 1.f : 0.f);
      }
      // off-diagonal blocks by block diagonals, T_ij = T_ii sum_{k=j}^{i-1} A_ik T_kj; the
      // blocks of one diagonal are independent (their product chains interleave) and are
      // stored together before the next diagonal reads them.  fp32 MFMA 16x16x4: in step
      // s lane group g carries k = 4s + g of the sum, and k = 4g + s of the T_ii product,
      // whose B operand is then the accumulator element s of the same lane.
      gc_off_diagonal<3>(sh.r2.s.am, sh.r2.s.tf, r16, g4);
      gc_off_diagonal<2>(sh.r2.s.am, sh.r2.s.tf, r16, g4);
      gc_off_diagonal<1>(sh.r2.s.am, sh.r2.s.tf, r16, g4);
    } else {
      // tiles (ti >= tj) of (q_i . k_j): wave 1 takes 0, 3, 6, 9; wave 2 1, 4, 7; wave 3 2, 5, 8
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int q = wave - 1 + 3 * n;
        qk[n] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
        if (q < 10) {
          const int ti = q < 1 ? 0 : (q < 3 ? 1 : (q < 6 ? 2 : 3));
          const int tj = q - ti * (ti + 1) / 2;
          gc_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc = gc_mma(gc_ld8(&sh.qc[16 * ti + r16][32 * s + 8 * g4]),
                         gc_ld8(&sh.r1.kc[16 * tj + r16][32 * s + 8 * g4]), acc);
          const int i0 = 16 * ti + 4 * g4, jj = 16 * tj + r16;
          const float4 rq = *reinterpret_cast<const float4*>(&sh.rqv[i0]);
          const float4 gi = *reinterpret_cast<const float4*>(&sh.gcv[i0]);
          const float rqa[4] = {rq.x, rq.y, rq.z, rq.w}, gia[4] = {gi.x, gi.y, gi.z, gi.w};
          const float rkj = sh.rkv[jj], gj = sh.gcv[jj];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            qk[n][j] = jj <= i0 + j ? (acc[j] * rqa[j] * rkj) * qscale * __expf(gia[j] - gj) : 0.f;
        }
      }
    }
    __syncthreads();   // A, k (row layout) consumed; Tm complete
    if (wave > 0) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int q = wave - 1 + 3 * n;
        if (q < 10) {
          const int ti = q < 1 ? 0 : (q < 3 ? 1 : (q < 6 ? 2 : 3));
          const int tj = q - ti * (ti + 1) / 2;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const __bf16 hi = (__bf16)qk[n][j];
            sh.r1.in[0][16 * ti + 4 * g4 + j][16 * tj + r16] = gc_bits(hi);
            sh.r1.in[1][16 * ti + 4 * g4 + j][16 * tj + r16] = gc_bits((__bf16)(qk[n][j] - (float)hi));
          }
        }
      }
      // upper tiles (0, 1) and (2, 3) fall inside the 32-wide k steps of the O product
      if (wave == 1) {
        const int tr = lane < 32 ? 0 : 2, rr = (lane & 31) >> 1, half = lane & 1;
        const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          *reinterpret_cast<u32x4_t*>(&sh.r1.in[p][16 * tr + rr][16 * (tr + 1) + 8 * half]) = z;
        }
      }
    }
    // Tm diag(rk beta e^gc) and Tm diag(beta), hi / lo (thread = row, 16 columns)
    {
      const int i = tid >> 2, cb = tid & 3, c0 = 16 * cb;
      const bool live = cb <= (i >> 4);
      float tv[16];
#pragma unroll
      for (int c4 = 0; c4 < 16; c4 += 4) {
        const float4 f = live ? *reinterpret_cast<const float4*>(&sh.r2.s.tf[i][c0 + c4])
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        tv[c4] = f.x; tv[c4 + 1] = f.y; tv[c4 + 2] = f.z; tv[c4 + 3] = f.w;
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const float* f = m == 0 ? sh.fwv : sh.btv;
#pragma unroll
        for (int c8 = 0; c8 < 16; c8 += 8) {
          const gc_f32x4 fa = *reinterpret_cast<const gc_f32x4*>(f + c0 + c8);
          const gc_f32x4 fb = *reinterpret_cast<const gc_f32x4*>(f + c0 + c8 + 4);
          gc_f32x4 p, q;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[j] = tv[c8 + j] * fa[j];
            q[j] = tv[c8 + 4 + j] * fb[j];
          }
          gc_bf16x8 hi, lo;
          gc_split(p, q, hi, lo);
          *reinterpret_cast<gc_bf16x8*>(&sh.r3.tm[2 * m][i][c0 + c8]) = hi;
          *reinterpret_cast<gc_bf16x8*>(&sh.r3.tm[2 * m + 1][i][c0 + c8]) = lo;
        }
      }
    }
    __syncthreads();
    // ================= W^T = K^T (Tm diag(rk beta e^gc))^T, stored as -W =================
    // wave w: key blocks 2w, 2w + 1 x the 4 token blocks (k steps limited by Tm's triangle)
    {
      gc_f32x4 acc[2][4];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) acc[c][ib] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int s = 0; s <= (ib >> 1); ++s) {
          const gc_bf16x8 bh = gc_ld8(&sh.r3.tm[0][16 * ib + r16][32 * s + 8 * g4]);
          const gc_bf16x8 bl = gc_ld8(&sh.r3.tm[1][16 * ib + r16][32 * s + 8 * g4]);
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const gc_bf16x8 av = gc_ld8(&sh.kt[32 * wave + 16 * c + r16][32 * s + 8 * g4]);
            acc[c][ib] = gc_mma(av, bh, acc[c][ib]);
            acc[c][ib] = gc_mma(av, bl, acc[c][ib]);
          }
        }
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          uint16_t hb[4], lb[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x = -acc[c][ib][j];
            const __bf16 hi = (__bf16)x;
            hb[j] = gc_bits(hi);
            lb[j] = gc_bits((__bf16)(x - (float)hi));
          }
          const int i = 16 * ib + r16, k0 = 32 * wave + 16 * c + 4 * g4;
          *reinterpret_cast<uint2*>(&sh.r2.w[0][i][k0]) =
              make_uint2(hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16));
          *reinterpret_cast<uint2*>(&sh.r2.w[1][i][k0]) =
              make_uint2(lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16));
        }
    }
    __syncthreads();
    // ================= V' = Tm diag(beta) V - W S (this wave's value columns) =================
    gc_bf16x8 sth[4][2], stl[4][2];   // hi / lo of S as B operands, k-step s = keys 32s .. 32s+31
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int u = 0; u < 2; ++u) gc_split(st[2 * s][u], st[2 * s + 1][u], sth[s][u], stl[s][u]);
    gc_f32x4 vn[4][2];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int u = 0; u < 2; ++u) vn[tb][u] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
    {
      gc_bf16x8 vb[2][2];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int u = 0; u < 2; ++u) vb[s][u] = gc_ld8(&sh.vt[vcol + 16 * u + r16][32 * s + 8 * g4]);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int s = 0; s <= (tb >> 1); ++s) {
          const gc_bf16x8 ah = gc_ld8(&sh.r3.tm[2][16 * tb + r16][32 * s + 8 * g4]);
          const gc_bf16x8 al = gc_ld8(&sh.r3.tm[3][16 * tb + r16][32 * s + 8 * g4]);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            vn[tb][u] = gc_mma(ah, vb[s][u], vn[tb][u]);
            vn[tb][u] = gc_mma(al, vb[s][u], vn[tb][u]);
          }
        }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint16_t* rh = &sh.r2.w[0][16 * tb + r16][32 * s + 4 * g4];
          const uint16_t* rl = &sh.r2.w[1][16 * tb + r16][32 * s + 4 * g4];
          const gc_bf16x8 ah = gc_ld44(rh, rh + 16), al = gc_ld44(rl, rl + 16);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            vn[tb][u] = gc_mma(ah, sth[s][u], vn[tb][u]);
            vn[tb][u] = gc_mma(ah, stl[s][u], vn[tb][u]);
            vn[tb][u] = gc_mma(al, sth[s][u], vn[tb][u]);
          }
        }
    }
    // V' and diag(rk e^(gc_63 - gc)) V' as B operands over tokens (k step s2 = tokens
    // 32 s2 .. 32 s2 + 31, accumulator row order)
    gc_bf16x8 vph[2][2], vpl[2][2], vqh[2][2], vql[2][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        gc_split(vn[2 * s2][u], vn[2 * s2 + 1][u], vph[s2][u], vpl[s2][u]);
        gc_f32x4 p, q;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p[j] = vn[2 * s2][u][j] * sh.f7v[32 * s2 + 4 * g4 + j];
          q[j] = vn[2 * s2 + 1][u][j] * sh.f7v[32 * s2 + 16 + 4 * g4 + j];
        }
        gc_split(p, q, vqh[s2][u], vql[s2][u]);
      }
    __syncthreads();   // Tm and W consumed: the O staging may overwrite them
    // ================= O = diag(rq s e^gc) Q S + (masked s q.k decay) V' =================
    {
      gc_f32x4 ov[4][2];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int u = 0; u < 2; ++u) ov[ib][u] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint16_t* rq = &sh.qc[16 * ib + r16][32 * s + 4 * g4];
          const gc_bf16x8 aq = gc_ld44(rq, rq + 16);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            ov[ib][u] = gc_mma(aq, sth[s][u], ov[ib][u]);
            ov[ib][u] = gc_mma(aq, stl[s][u], ov[ib][u]);
          }
        }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 16 * ib + 4 * g4 + j;
          const float rs = sh.rqv[i] * qscale * sh.egv[i];
          ov[ib][0][j] *= rs;
          ov[ib][1][j] *= rs;
        }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int s2 = 0; s2 <= (ib >> 1); ++s2) {
          const uint16_t* rh = &sh.r1.in[0][16 * ib + r16][32 * s2 + 4 * g4];
          const uint16_t* rl = &sh.r1.in[1][16 * ib + r16][32 * s2 + 4 * g4];
          const gc_bf16x8 ah = gc_ld44(rh, rh + 16), al = gc_ld44(rl, rl + 16);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            ov[ib][u] = gc_mma(ah, vph[s2][u], ov[ib][u]);
            ov[ib][u] = gc_mma(ah, vpl[s2][u], ov[ib][u]);
            ov[ib][u] = gc_mma(al, vph[s2][u], ov[ib][u]);
          }
        }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int j = 0; j < 4; ++j) sh.r3.o[16 * ib + 4 * g4 + j][vcol + 16 * u + r16] = ov[ib][u][j];
    }
    // ================= S <- e^gc_63 S + K^T diag(rk e^(gc_63 - gc)) V' =================
    {
      const float elast = sh.egv[GC_C - 1];
#pragma unroll
      for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) st[kb][u] *= elast;
#pragma unroll
      for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const uint16_t* rk = &sh.kt[16 * kb + r16][32 * s2 + 4 * g4];
          const gc_bf16x8 ak = gc_ld44(rk, rk + 16);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            st[kb][u] = gc_mma(ak, vqh[s2][u], st[kb][u]);
            st[kb][u] = gc_mma(ak, vql[s2][u], st[kb][u]);
          }
        }
    }
    __syncthreads();   // O complete; every chunk buffer consumed
    // the next chunk's inputs, issued unconditionally (after the last chunk: rows clamped
    // into the call, never used) so the wait counts of the norm below stay exact
    {
      const uint32_t cb = (uint32_t)(t0 + GC_C) * P2;
#pragma unroll
      for (int n = 0; n < GC_ITEMS; ++n)
#pragma unroll
        for (int r = 0; r < 7; ++r) raw[n][r] = gc_bload(prs, roff[n] + cb + (uint32_t)r * P2);
      braw = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(prs, boff + cb, 0, 0);
      araw = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(prs, boff + cb + 2u * a.Hv, 0, 0);
    }
    // ================= gated RMSNorm, 16 threads per token, 8 columns each =================
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int i = 16 * n + (tid >> 4), part = tid & 15, t = t0 + i;
      const float4 oa = *reinterpret_cast<const float4*>(&sh.r3.o[i][part * 8]);
      const float4 ob = *reinterpret_cast<const float4*>(&sh.r3.o[i][part * 8 + 4]);
      const float ovf[8] = {oa.x, oa.y, oa.z, oa.w, ob.x, ob.y, ob.z, ob.w};
      float ovs[8], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {   // the core output is a bf16 tensor
        const uint32_t pv = gc_pack(ovf[e], ovf[e + 1]);
        ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gc_bf16x2, pv),
                                             __builtin_bit_cast(gc_bf16x2, pv), ss, false);
        ovs[e] = __uint_as_float(pv << 16);
        ovs[e + 1] = __uint_as_float(pv & 0xffff0000u);
      }
      ss = gc_row16_sum(ss);
      const float rr = rsqrtf(ss / (float)GL_DK + a.eps);
      const uint32_t zd[4] = {zreg[n][0], zreg[n][1], zreg[n][2], zreg[n][3]};
      uint32_t od[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float y2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int ee = e + u;
          const float z = __uint_as_float(ee & 1 ? zd[ee >> 1] & 0xffff0000u : zd[ee >> 1] << 16);
          y2[u] = gc_rbf(nwf[ee] * gc_rbf(ovs[ee] * rr)) * silu_g(z);
        }
        od[e >> 1] = gc_pack(y2[0], y2[1]);
      }
      if (t < a.T)
        *reinterpret_cast<uint4*>(a.out + ((size_t)b * a.T + t) * a.value_dim + (size_t)h * GL_DK +
                                  part * 8) = make_uint4(od[0], od[1], od[2], od[3]);
    }
  }
  // ---- final state in the written half; final K-1 raw inputs in the window ----
  {
    float* sf = st_io;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sf[(size_t)(16 * kb + 4 * g4 + j) * GL_DK + vcol + 16 * u + r16] = st[kb][u][j];
    for (int i = tid; i < Km1 * GL_CH; i += 256) {
      const int r = i / GL_CH, lc = i % GL_CH;
      if (lc >= 2 * GL_DK || write_qk) {
        const int c = gc_chan(a, hk, h, lc);
        a.win[(win_b + wbase + r) * a.C + c] = a.proj[((size_t)b * a.T + a.T - Km1 + r) * a.P + c];
      }
    }
  }
}

}  // namespace lollm

using namespace lollm;

LOLLM_API int lollm_gdn_layer_chunked(const void* proj, long long proj_stride, const void* conv_w,
                                      const float* A_log, const float* dt_bias, const void* norm_w,
                                      void* win, const int32_t* conv_off, int win_rows, float* rec,
                                      const int32_t* rec_half, void* rep, const int32_t* replay,
                                      int slots, int fresh, void* out, int B, int T, int Hk, int Hv,
                                      int Dk, int Dv, int conv_kernel, float eps, void* stream) {
  if (!proj || !conv_w || !A_log || !dt_bias || !norm_w || !win || !conv_off || !rec ||
      !rec_half || !rep || !replay || !out)
    return LOLLM_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return LOLLM_EINVAL;
  if (Dk != GL_DK || Dv != GL_DK || conv_kernel != 4) return LOLLM_EUNSUPPORTED;
  if (win_rows < conv_kernel - 1 || slots < 1) return LOLLM_EINVAL;
  // the long-call placement: no per-position snapshots, the window half too short to
  // hold the whole call (so only the final K-1 raw rows are written)
  if (T <= slots || conv_kernel - 1 + T <= win_rows || T < conv_kernel - 1) return LOLLM_EUNSUPPORTED;
  const int key_dim = Hk * Dk, value_dim = Hv * Dv, C = 2 * key_dim + value_dim;
  if (proj_stride < (long long)C + value_dim + 2 * Hv || proj_stride % 8) return LOLLM_EINVAL;
  if ((long long)T * proj_stride * 2 >= (1LL << 31)) return LOLLM_EUNSUPPORTED;   // 32-bit row offsets
  GdnLayerArgs a;
  a.proj = (const uint16_t*)proj; a.conv_w = (const uint16_t*)conv_w; a.A_log = A_log;
  a.dt_bias = dt_bias; a.norm_w = (const uint16_t*)norm_w; a.win = (uint16_t*)win;
  a.conv_off = conv_off; a.rec = rec; a.rec_half = rec_half; a.rep = (uint8_t*)rep;
  a.replay = replay; a.out = (uint16_t*)out;
  a.P = proj_stride; a.T = T; a.Hk = Hk; a.Hv = Hv; a.C = C; a.key_dim = key_dim;
  a.value_dim = value_dim; a.K = conv_kernel; a.W = win_rows; a.S = slots; a.fresh = fresh ? 1 : 0;
  a.eps = eps;
  const int rc = gdn_long_call_prologue(a, B, (hipStream_t)stream);
  if (rc != LOLLM_OK) return rc;
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(B * Hv), dim3(256), 0, (hipStream_t)stream, a);
  return launch_status();
}

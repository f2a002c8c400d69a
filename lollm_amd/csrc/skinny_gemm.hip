// Weight-streaming GEMM for the few-row projections of the speculative step (gfx950):
// C[M, N] = A[M, K] W[N, K]^T with M <= 64 (the 1 + k verify positions of B sequences,
// or the B draft positions), bf16 in, fp32 accumulate, bf16 out.  Every weight byte is
// read once per call, so the kernel is an HBM stream of W with 64 MACs per weight at
// most; it replaces F.linear for in_proj / out_proj / q,k,v / o_proj / gate_up / down /
// lm_head / MTP fc (src/qwen3_5/blocks.py:199-236,288-342, modeling_qwen3_5.py:73-99,
// mtp.py:61-73) when the rows are few.
//
// Weight layout (tiled once at load by lollm_gemm_tile_weights): 1 KB blocks in the
// order the 16x16x32 bf16 MFMA consumes them.  Block (t, s) -- n-tile t (16 rows),
// k-step s (32 k) -- sits at element offset (t * K / 32 + s) * 512, and lane L = 16 g + r
// of the block holds row 16 t + r, k = 32 s + 8 g .. + 8, so a block is one coalesced
// 1 KB read that lands exactly as a wave's MFMA A operand.  The SwiGLU layout interleaves
// gate and up rows 8 by 8 (tile t = gate rows 8t..8t+7, then up rows 8t..8t+7) so a lane
// and its partner 32 lanes away hold gate and up of the same output columns.
//
// Work decomposition: a group = 64 output columns (4 n-tiles; 96 where that leaves no
// group cut, gemm_group_tiles), a unit = (group, 128-k stage).  Units are laid end to end group-major and dealt out in equal contiguous ranges
// to a fixed grid (one workgroup per CU), so every workgroup streams the same number of
// weight bytes whatever N is (N / 64 groups over 256 CUs would run uneven rounds).  Two
// kernels: gemm_ksplit_kernel for at most 32 rows (operands straight to registers, each
// wave one k-step of every unit), gemm_stream_kernel for 33..64 rows (warp-specialised:
// DMA loader waves stream weights and activations into LDS rings, MFMA waves consume
// them; see each).  A group one workgroup covers whole is stored directly (with the
// epilogue); a group cut between workgroups leaves an fp32 piece in slot w + group: in
// accumulator order when gemm_fixup_kernel merges it with one float4 per thread over a
// (group, m-tile) grid, row major when gemm_norm_kernel merges it row by row.  (Merging
// in the last-arriving workgroup instead would need device-scope release / acquire
// fences, which write back and invalidate the XCD's L2 -- measured 3-10x slower here
// than the second launch.)
#include "common.h"

namespace lollm {

typedef __bf16 gm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float gm_f32x4 __attribute__((ext_vector_type(4)));

constexpr int GM_KC = 128;                  // k per unit
constexpr int GM_KS = GM_KC / 32;           // MFMA k-steps per unit
constexpr int GM_COLS = 64;                 // output columns (tiled rows) per group
constexpr int GM_PITCH = GM_KC * 2 + 16;    // padded bytes per activation row in LDS
constexpr int GM_P = 4;                     // weight units in flight per wave
constexpr int GM_MAXW = 1024;               // grid limit (piece table)
constexpr int GM_PB = 8;                    // piece loads a merge issues together

enum { GM_EPI_NONE = 0, GM_EPI_SWIGLU = 1, GM_EPI_ARGMAX = 2, GM_EPI_LOGITS = 3 };

// Row argmax without the logits (lollm_gemm_argmax): each (row, 16-column n-tile) keeps
// the packed maximum ((order key of the bf16 value) << 32 | ~column), so the highest
// value wins and ties go to the lowest column -- the rule of the sampler's greedy rows.
__device__ __forceinline__ uint64_t gm_key(float v, int col) {
  const uint32_t b = f32_to_bf16(v);
  const uint32_t o = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return ((uint64_t)o << 32) | (0xFFFFFFFFu - (uint32_t)col);
}
__device__ __forceinline__ uint64_t gm_max_xor(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, 64), hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o > v ? o : v;
}

struct GemmArgs {
  const uint16_t* A;     // (M, K) activations, row stride lda
  const uint16_t* Wt;    // tiled weights
  uint16_t* C;           // (M, ldc)
  float* part;           // (nw + G) pieces of (16 MT) x 64 fp32
  long long lda, ldc;
  int M, N, K, G, SK, nw, epi, U;
  int rowmajor;          // piece layout: 0 = accumulator order (float4 (i, wave, lane)), 1 = row major
  uint64_t* am;          // GM_EPI_ARGMAX: (M, N / 16) packed row maxima per n-tile
  // GM_EPI_LOGITS: the bf16 logits with the repetition penalty applied in place, and per
  // row the maximum order key of the stored values in 2 nw slots (row stride rmax_ld):
  // slot w = the groups workgroup w finished whole, slot nw + w = the cut group whose
  // last unit workgroup w holds (merged by the fixup kernel; 0 where there is none)
  uint16_t* rmax;
  long long rmax_ld;
  const uint32_t* seen;  // (M / T, seen_words) bitmaps of the penalised tokens, or null
  int seen_words;
  const int32_t* extra;  // extra penalised tokens: row m = (s, t) also counts
  int extra_stride;      //   extra[s * extra_stride + j] for j < n_extra0 + t
  int n_extra0, T;
  float pen;
};

// The penalty context of one row for GM_EPI_LOGITS: its extra penalised tokens (at most
// GM_MAXEX, checked on the host); the seen-bitmap word of a column goes with it.
constexpr int GM_MAXEX = 8;
struct GmRowEx {
  int n;
  int32_t ex[GM_MAXEX];
};

__device__ __forceinline__ void gm_row_ex(const GemmArgs& a, int m, GmRowEx& r) {
  r.n = 0;
  if (!a.seen || !a.extra) return;
  const int mm = m < a.M ? m : a.M - 1;
  const int sq = mm / a.T, t = mm - sq * a.T;
  r.n = a.n_extra0 + t;
  const int32_t* ex = a.extra + (size_t)sq * a.extra_stride;
#pragma unroll
  for (int j = 0; j < GM_MAXEX; ++j) r.ex[j] = j < r.n ? ex[j] : -1;
}

// bits col .. col + 3 (col % 4 == 0) of row m's seen bitmap, in bits 0..3
__device__ __forceinline__ uint32_t gm_seen4(const GemmArgs& a, int m, int col) {
  if (!a.seen) return 0u;
  const int mm = m < a.M ? m : a.M - 1;
  const int sq = mm / a.T;
  return a.seen[(size_t)sq * a.seen_words + (col >> 5)] >> (col & 31);
}

// The bf16 logits of columns col .. col + 3 of a row (output tile values v) with the
// repetition penalty of src/generate.py:18-22 applied where the token is in the row's
// context (seen bits w, extra tokens r): bf16(v), then for a penalised token
// y = x > 0 ? x / pen : x * pen in fp32 rounded once to bf16 -- the bits
// lollm_repetition_penalty gives on the stored logits.
__device__ __forceinline__ void gm_logits4(const GemmArgs& a, const float* v, int col, uint32_t w,
                                           const GmRowEx& r, uint32_t* bits) {
#pragma unroll
  for (int e = 0; e < 4; ++e) bits[e] = f32_to_bf16(v[e]);
  if (!a.seen) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    bool p = (w >> e) & 1u;
#pragma unroll
    for (int j = 0; j < GM_MAXEX; ++j) p |= j < r.n && r.ex[j] == col + e;
    if (p) {
      const float x = __uint_as_float(bits[e] << 16);
      bits[e] = f32_to_bf16(x > 0.f ? x / a.pen : x * a.pen);
    }
  }
}

__device__ __forceinline__ uint32_t gm_ord16(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

// Row-maximum slots of a GM_EPI_LOGITS call, GM_RM_SLOTS per workgroup and row: in the
// main kernels slot GM_RM_SLOTS w + v holds the maximum order key over the whole groups
// wave v of workgroup w stored (the k-split kernel's 4 waves, the stream kernel's 2 column
// halves, the rest 0); slot GM_RM_SLOTS nw + w that of the cut group whose last unit
// workgroup w holds (written by the fixup kernel; 0 where there is none).  Every slot
// of rows < M is written by every call, so nothing needs clearing.
constexpr int GM_RM_SLOTS = 4;

__device__ __forceinline__ void gm_rowmax_put(const GemmArgs& a, int m, int slot, uint32_t x) {
  if (m < a.M) a.rmax[(size_t)m * a.rmax_ld + slot] = (uint16_t)x;
}

// lanes l and l ^ 16, l ^ 32, l ^ 48 hold the same row: their maximum
__device__ __forceinline__ uint32_t gm_rowmax_lanes(uint32_t x) {
  x = max(x, (uint32_t)__shfl_xor((int)x, 16, 64));
  return max(x, (uint32_t)__shfl_xor((int)x, 32, 64));
}

__device__ __forceinline__ void gm_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float gm_silu_bf16(float g) {
  // the unfused path rounds the GEMM output, silu's output and the product to bf16
  const float gr = round_bf16(g);
  return round_bf16(gr / (1.f + __expf(-gr)));
}

__device__ __forceinline__ int gm_begin(int U, int w, int nw) { return (int)((long long)U * w / nw); }
__device__ __forceinline__ int gm_owner(int U, int u, int nw) {
  return (int)(((long long)(u + 1) * nw - 1) / U);
}

__global__ void gemm_tile_kernel(const uint16_t* __restrict__ W, uint16_t* __restrict__ Wt, int N,
                                 int K, int mode) {
  const size_t blk = blockIdx.x;
  const int ks = K / 32;
  const int t = (int)(blk / ks), s = (int)(blk % ks);
  const int L = threadIdx.x, r = L & 15, g = L >> 4;
  int src = 16 * t + r;
  if (mode == GM_EPI_SWIGLU) src = (r < 8 ? 0 : N / 2) + 8 * t + (r & 7);
  const uint4 v = *reinterpret_cast<const uint4*>(W + (size_t)src * K + 32 * s + 8 * g);
  *reinterpret_cast<uint4*>(Wt + blk * 512 + L * 8) = v;
}

// The product for 33..64 rows, warp-specialised.  Waves 4 and 5 only stream weights:
// each copies its half of a unit's weight blocks (2 n-tiles x 4 k-steps, 1 KB each, for
// 64-column groups)
// straight into LDS with 16-byte DMA loads (global_load_lds_dwordx4, non-temporal) into a
// ring of GS_WSLOTS slots, GS_WSLOTS - 1 units ahead (3 slots: measured 1-3% faster per
// launch than 4 to 7 in the decode step -- a shallower DMA queue per CU queues less on
// the memory side -- and 2 slots 7% slower); wave 6 copies the unit's 64-row
// activation tile (128 k) the same way into a ring of GS_ASLOTS slots.  Only these
// three waves wait on vmcnt, each for its own oldest unit with a fixed count, so the
// weight stream never waits for anything else (in the register-ring kernel every wait
// for an activation or a weight also waited for all older loads, in issue order, and
// the compiler added full drains at the loop head).  Waves 0-3 read both MFMA operands
// from LDS in a 2 x 2 arrangement -- wave (wn, wm) owns n-tiles 2 wn, 2 wn + 1 and m-tiles
// 2 wm, 2 wm + 1 of the group -- with one accumulator per k-step of the unit (q = k-step
// mod 4), added in the order 0, 1, 2, 3 at the group's end: exactly the sums and order of
// gemm_ksplit_kernel, whose wave q accumulates k-steps 4 s + q, so a row's bits do not
// depend on how many rows share the call (1..32 rows run that kernel, 33..64 this one).
// One barrier per unit: past it the unit has
// landed and every consumer has finished the previous unit, whose slots the loaders
// refill.  Activation rows sit in LDS without padding, the 16-byte chunk c of row r at
// chunk position c ^ (r & 15) (the DMA writes a wave's 1 KB contiguously, so the loaders
// pick each lane's source chunk to produce that layout; the consumers' 16 rows of one
// chunk then hit 16 different bank groups).  Rows past M re-read the last row.  Past
// the range's end the loaders refetch its last unit into the free slot, so their wait
// counts stay exact.  Measured 3-8% faster at 64 rows than that register-ring kernel
// (weights and activations in a 4-unit register ring, activations staged into LDS by
// the MFMA waves) on every projection shape of the 8B-class verify pass.
typedef __attribute__((address_space(1))) void gs_global_t;
typedef __attribute__((address_space(3))) void gs_lds_t;
constexpr int GS_WSLOTS = 3;
constexpr int GS_ASLOTS = 3;
constexpr int GS_SLOT = 16384;
constexpr int GS_THREADS = 448;
constexpr int GS_NT = 2;                    // cache policy of the weight DMA: non-temporal

// GM_EPI_LOGITS: sw = gm_seen4 of the lane's columns (0 when the caller has no penalty
// context ready: it is then loaded here), rx = the row's extra tokens, rm = the lane's
// row maximum so far.
template <int NT>
__device__ __forceinline__ void gs_emit_tile(const GemmArgs& a, const gm_f32x4& v, int i, int j,
                                             int g, bool whole, int w, int lane, uint32_t& rm,
                                             uint32_t sw, const GmRowEx& rx) {
  const int l16 = lane & 15, g4 = lane >> 4;
  const int m = 16 * i + l16;
  const int t = NT * g + j;                  // n-tile of the tiled weight
  if (whole) {
    if (a.epi == GM_EPI_LOGITS) {
      if (m < a.M) {
        const int col = 16 * t + 4 * g4;
        const float vv[4] = {v[0], v[1], v[2], v[3]};
        uint32_t b[4];
        gm_logits4(a, vv, col, sw, rx, b);
#pragma unroll
        for (int e = 0; e < 4; ++e) rm = max(rm, gm_ord16(b[e]));
        *reinterpret_cast<uint2*>(a.C + (size_t)m * a.ldc + col) =
            make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
      }
    } else if (a.epi == GM_EPI_ARGMAX) {
      const int col = 16 * t + 4 * g4;
      uint64_t best = gm_key(v[0], col);
#pragma unroll
      for (int e = 1; e < 4; ++e) {
        const uint64_t k2 = gm_key(v[e], col + e);
        best = k2 > best ? k2 : best;
      }
      best = gm_max_xor(best, 16);
      best = gm_max_xor(best, 32);
      if (g4 == 0 && m < a.M) a.am[(size_t)m * (a.N / 16) + t] = best;
    } else if (a.epi == GM_EPI_SWIGLU) {
      float other[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) other[e] = __shfl_xor(v[e], 32, 64);
      if (g4 < 2 && m < a.M) {
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = round_bf16(gm_silu_bf16(v[e]) * round_bf16(other[e]));
        const int col = 8 * t + 4 * g4;
        *reinterpret_cast<uint2*>(a.C + (size_t)m * a.ldc + col) =
            make_uint2((uint32_t)f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16),
                       (uint32_t)f32_to_bf16(y[2]) | ((uint32_t)f32_to_bf16(y[3]) << 16));
      }
    } else if (m < a.M) {
      const int col = 16 * t + 4 * g4;
      *reinterpret_cast<uint2*>(a.C + (size_t)m * a.ldc + col) =
          make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                     (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
    }
  } else if constexpr (NT == 4) {
    // the piece of a cut group in the layout the merge kernels read: (16 mt) x 64 fp32
    // with mt = ceil(M / 16) m-tiles, so an m-tile made only of padding rows is skipped
    // (wider groups are never cut: the host gives them a grid that divides them)
    const int mt = (a.M + 15) / 16;
    if (i >= mt) return;
    float* pp = a.part + ((size_t)w + g) * ((size_t)mt * 16 * GM_COLS);
    const size_t off = a.rowmajor ? (size_t)m * GM_COLS + 16 * j + 4 * g4
                                  : (((size_t)i * 4 + j) * 64 + lane) * 4;
    *reinterpret_cast<float4*>(pp + off) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// NT n-tiles per group: 4 (64 columns) in general; 6 (96 columns) where 96-column groups
// divide evenly over the grid and 64-column ones would be cut (the MLP gate|up of the
// 4096-hidden model: 256 groups, one per CU, so no merge launch follows; the attention
// q|gate|k|v: 192).  A wide unit is 24 KB of weights against the same 16 KB activation
// tile.  Each output
// tile accumulates the same k-steps in the same order for either width, so a group
// finished by one workgroup has the same bits at both widths.
template <int NT>
__global__ __launch_bounds__(GS_THREADS) void gemm_stream_kernel(GemmArgs a) {
  constexpr int WSLOTS = GS_WSLOTS;
  constexpr int WSLOT = NT * GM_KS * 1024;   // bytes of one unit's weight blocks
  constexpr int HALF = NT / 2;               // n-tiles per loader wave and per MFMA wave
  static_assert(NT % 2 == 0 && WSLOTS * WSLOT + GS_ASLOTS * GS_SLOT <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[WSLOTS * WSLOT + GS_ASLOTS * GS_SLOT];
  unsigned char* wring = lds;
  unsigned char* aring = lds + WSLOTS * WSLOT;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int w = blockIdx.x;
  const int u0 = gm_begin(a.U, w, a.nw), u1 = gm_begin(a.U, w + 1, a.nw);
  if (u0 >= u1) {                            // the whole workgroup: no barrier is left waiting
    if (a.epi == GM_EPI_LOGITS && threadIdx.x < 64) {
#pragma unroll
      for (int v = 0; v < GM_RM_SLOTS; ++v) gm_rowmax_put(a, threadIdx.x, GM_RM_SLOTS * w + v, 0);
      gm_rowmax_put(a, threadIdx.x, GM_RM_SLOTS * a.nw + w, 0);
    }
    return;
  }
  const int kt = a.K / 32;
  if (wave == 4 || wave == 5) {
    const int lw = wave - 4;
    auto issue = [&](int u) {
      const int uu = u < u1 ? u : u1 - 1;
      const int g = uu / a.SK, st = uu - g * a.SK;
      unsigned char* sb = wring + ((u - u0) % WSLOTS) * WSLOT;
#pragma unroll
      for (int jj = 0; jj < HALF; ++jj) {
        const int j = HALF * lw + jj;
        const uint16_t* src = a.Wt + ((size_t)(NT * g + j) * kt + (size_t)st * GM_KS) * 512 + lane * 8;
#pragma unroll
        for (int q = 0; q < GM_KS; ++q)
          __builtin_amdgcn_global_load_lds((gs_global_t*)(src + q * 512),
                                           (gs_lds_t*)(sb + (j * GM_KS + q) * 1024), 16, 0, GS_NT);
      }
    };
#pragma unroll
    for (int p = 0; p < WSLOTS - 1; ++p) issue(u0 + p);
    for (int u = u0; u < u1; ++u) {
      // unit u has landed once at most WSLOTS - 2 younger units (HALF * 4 DMAs each) remain
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"((WSLOTS - 2) * HALF * GM_KS) : "memory");
      issue(u + WSLOTS - 1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  if (wave == 6) {
    auto issue = [&](int u) {
      const int uu = u < u1 ? u : u1 - 1;
      const int k0 = (uu % a.SK) * GM_KC;
      unsigned char* sb = aring + ((u - u0) % GS_ASLOTS) * GS_SLOT;
#pragma unroll
      for (int d = 0; d < 16; ++d) {
        const int r = 4 * d + (lane >> 4), p = lane & 15, c = p ^ (r & 15);
        const int rr = r < a.M ? r : a.M - 1;
        __builtin_amdgcn_global_load_lds((gs_global_t*)(a.A + (size_t)rr * a.lda + k0 + c * 8),
                                         (gs_lds_t*)(sb + d * 1024), 16, 0, 0);
      }
    };
#pragma unroll
    for (int p = 0; p < GS_ASLOTS - 1; ++p) issue(u0 + p);
    for (int u = u0; u < u1; ++u) {
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"((GS_ASLOTS - 2) * 16) : "memory");
      issue(u + GS_ASLOTS - 1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  const int wn = wave & 1, wm = wave >> 1, l16 = lane & 15, g4 = lane >> 4;
  gm_f32x4 acc[GM_KS][2][HALF];
#pragma unroll
  for (int q = 0; q < GM_KS; ++q)
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int jj = 0; jj < HALF; ++jj) acc[q][ii][jj] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
  bool whole_from_start = (u0 % a.SK) == 0;
  uint32_t rm[2] = {0u, 0u};                 // GM_EPI_LOGITS: row maxima (order keys)
  // GM_EPI_LOGITS with a penalty: each row's extra tokens, and the seen words of the
  // group's columns loaded at the group's first unit, long before its epilogue needs them
  GmRowEx rx[2];
  uint32_t sw[2][HALF];
#pragma unroll
  for (int ii = 0; ii < 2; ++ii) {
    gm_row_ex(a, 16 * (2 * wm + ii) + l16, rx[ii]);
#pragma unroll
    for (int jj = 0; jj < HALF; ++jj) sw[ii][jj] = 0u;
  }
  for (int u = u0; u < u1; ++u) {
    if (a.epi == GM_EPI_LOGITS && a.seen && (u == u0 || u % a.SK == 0)) {
      const int g = u / a.SK;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int jj = 0; jj < HALF; ++jj)
          sw[ii][jj] = gm_seen4(a, 16 * (2 * wm + ii) + l16, 16 * (NT * g + HALF * wn + jj) + 4 * g4);
    }
    // this wave's reads of the previous unit are complete before the loaders may refill it
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const unsigned char* wb = wring + ((u - u0) % WSLOTS) * WSLOT;
    const unsigned char* ab = aring + ((u - u0) % GS_ASLOTS) * GS_SLOT;
#pragma unroll
    for (int q = 0; q < GM_KS; ++q) {
      gm_bf16x8 wf[HALF], af[2];
#pragma unroll
      for (int jj = 0; jj < HALF; ++jj)
        wf[jj] = *reinterpret_cast<const gm_bf16x8*>(wb + ((HALF * wn + jj) * GM_KS + q) * 1024 + lane * 16);
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int row = 16 * (2 * wm + ii) + l16, c = q * 4 + g4;
        af[ii] = *reinterpret_cast<const gm_bf16x8*>(ab + row * 256 + ((c ^ (row & 15)) * 16));
      }
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int jj = 0; jj < HALF; ++jj)
          acc[q][ii][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[jj], af[ii], acc[q][ii][jj], 0, 0, 0);
    }
    const int st = u % a.SK;
    if (st == a.SK - 1 || u == u1 - 1) {
      const int g = u / a.SK;
      const bool whole = whole_from_start && st == a.SK - 1;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int jj = 0; jj < HALF; ++jj) {
          gm_f32x4 fin = acc[0][ii][jj];
#pragma unroll
          for (int q = 1; q < GM_KS; ++q) fin += acc[q][ii][jj];
          gs_emit_tile<NT>(a, fin, 2 * wm + ii, HALF * wn + jj, g, whole, w, lane, rm[ii],
                           sw[ii][jj], rx[ii]);
#pragma unroll
          for (int q = 0; q < GM_KS; ++q) acc[q][ii][jj] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
        }
      whole_from_start = true;
    }
  }
  if (a.epi == GM_EPI_LOGITS) {
    // wave (wn, wm): slot wn of its 32 rows' column half, slot 2 + wn cleared
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const uint32_t x = gm_rowmax_lanes(rm[ii]);
      if (g4 == 0) {
        const int m = 16 * (2 * wm + ii) + l16;
        gm_rowmax_put(a, m, GM_RM_SLOTS * w + wn, x);
        gm_rowmax_put(a, m, GM_RM_SLOTS * w + 2 + wn, 0);
      }
    }
    if (wave == 0) gm_rowmax_put(a, lane, GM_RM_SLOTS * a.nw + w, 0);
  }
}


// The same product for at most 32 rows: each wave takes one k-step of every unit for all
// NT n-tiles of the group, so it reads its MFMA operands straight from memory -- weights
// (NT blocks, one per n-tile) and activations (one 16-row x 64 B chunk per m-tile) -- into
// a register ring 4 units deep, with no LDS staging and no barrier in the unit loop.
// At a group's end the 4 waves' k-quarters are summed through LDS in a fixed order
// (wave 0 .. 3) and emitted as above, n-tile j by wave j % 4.  The activation chunks are half cache lines (every
// line is read by two waves), which costs more than the LDS staging at 64 rows; at 16
// and 32 rows, with one workgroup per CU, this form measured 3-10% faster.
template <int MT, int NT>
__global__ __launch_bounds__(256, 2) void gemm_ksplit_kernel(GemmArgs a) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  // the waves' partial sums at a group's end: (n-tile j, wave v, m-tile i) x 64 lanes
  __shared__ __attribute__((aligned(16))) gm_f32x4 red[NT * 4 * MT * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int w = blockIdx.x;
  const int u0 = gm_begin(a.U, w, a.nw), u1 = gm_begin(a.U, w + 1, a.nw);
  if (u0 >= u1) {
    if (a.epi == GM_EPI_LOGITS && tid < 64) {
#pragma unroll
      for (int v = 0; v < GM_RM_SLOTS; ++v) gm_rowmax_put(a, tid, GM_RM_SLOTS * w + v, 0);
      gm_rowmax_put(a, tid, GM_RM_SLOTS * a.nw + w, 0);
    }
    return;
  }
  const int kt = a.K / 32;
  const uint16_t* wlane = a.Wt + (size_t)wave * 512 + lane * 8;
  const uint16_t* alane[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int r = min(16 * i + l16, a.M - 1);   // padding rows re-read the last row
    alane[i] = a.A + (size_t)r * a.lda + 32 * wave + 8 * g4;
  }
  v4u wr[GM_P][NT], ar[GM_P][MT];
  // weights of unit u: n-tiles NT g + j, k-step 4 st + wave; activations: k-step 4 st + wave
  auto load = [&](v4u* dw, v4u* da, int u) {
    const int g = u / a.SK, st = u - g * a.SK;
    const uint16_t* p = wlane + ((size_t)NT * g * kt + (size_t)st * GM_KS) * 512;
#pragma unroll
    for (int j = 0; j < NT; ++j)
      dw[j] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p + (size_t)j * kt * 512));
#pragma unroll
    for (int i = 0; i < MT; ++i) da[i] = *reinterpret_cast<const v4u*>(alane[i] + st * GM_KC);
  };
  gm_f32x4 acc[NT][MT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[j][i] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
  // every load is issued unconditionally (units past the range re-read the last one) and
  // the slots are issued oldest first, so each unit waits only for its own slot
  const int ulast = u1 - 1;
#pragma unroll
  for (int p = 0; p < GM_P; ++p) {
    load(wr[p], ar[p], u0 + p < u1 ? u0 + p : ulast);
    __builtin_amdgcn_sched_barrier(0);
  }
  bool whole_from_start = (u0 % a.SK) == 0;
  uint32_t rm[MT];                            // GM_EPI_LOGITS: row maxima (order keys)
#pragma unroll
  for (int i = 0; i < MT; ++i) rm[i] = 0u;

  auto finish = [&](int g, bool whole) {
    gm_lds_barrier();   // the previous group's reads of red are done
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i) red[((j * 4 + wave) * MT + i) * 64 + lane] = acc[j][i];
    gm_lds_barrier();
#pragma unroll
    for (int j = wave; j < NT; j += 4) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        gm_f32x4 fin = red[((j * 4) * MT + i) * 64 + lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) fin += red[((j * 4 + v) * MT + i) * 64 + lane];
        uint32_t swk = 0u;
        GmRowEx rxk;
        rxk.n = 0;
        if (a.epi == GM_EPI_LOGITS && whole) {
          swk = gm_seen4(a, 16 * i + l16, 16 * (NT * g + j) + 4 * g4);
          gm_row_ex(a, 16 * i + l16, rxk);
        }
        gs_emit_tile<NT>(a, fin, i, j, g, whole, w, lane, rm[i], swk, rxk);
      }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[j][i] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
  };

#define GM_KUNIT(J)                                                                           \
  {                                                                                           \
    const int u = ub + (J);                                                                   \
    const bool livej = u < u1;                                                                \
    if (livej) {                                                                              \
      _Pragma("unroll") for (int j = 0; j < NT; ++j) {                                        \
        _Pragma("unroll") for (int i = 0; i < MT; ++i) {                                      \
          acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(                                \
              __builtin_bit_cast(gm_bf16x8, wr[J][j]), __builtin_bit_cast(gm_bf16x8, ar[J][i]), \
              acc[j][i], 0, 0, 0);                                                            \
        }                                                                                     \
      }                                                                                       \
    }                                                                                         \
    load(wr[J], ar[J], u + GM_P < u1 ? u + GM_P : ulast);                                     \
    if (livej) {                                                                              \
      const int st = u % a.SK;                                                                \
      if (st == a.SK - 1 || u == ulast) {                                                     \
        finish(u / a.SK, whole_from_start && st == a.SK - 1);                                 \
        whole_from_start = true;                                                              \
      }                                                                                       \
    }                                                                                         \
  }

  static_assert(GM_P == 4, "the unit loop is unrolled by 4");
  for (int ub = u0; ub < u1; ub += 4) {
    GM_KUNIT(0) GM_KUNIT(1) GM_KUNIT(2) GM_KUNIT(3)
  }
#undef GM_KUNIT
  if (a.epi == GM_EPI_LOGITS) {
    // wave v emitted n-tiles v, v + 4, ... of every row: slot v
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const uint32_t x = gm_rowmax_lanes(rm[i]);
      if (g4 == 0) gm_rowmax_put(a, 16 * i + l16, GM_RM_SLOTS * w + wave, x);
    }
    if (wave == 0) gm_rowmax_put(a, lane, GM_RM_SLOTS * a.nw + w, 0);
  }
}

// Merge the pieces of m-tile blockIdx.y of group blockIdx.x: the live piece slots are
// listed in LDS by one wave (ballots over the workgroups whose ranges touch the group;
// empty ranges leave no piece), then each thread sums one float4 (the one its lane
// held in the main kernel) over the pieces in slot order and applies the epilogue.
// Groups one workgroup finished are skipped.
__global__ __launch_bounds__(256) void gemm_fixup_kernel(GemmArgs a) {
  __shared__ int live[GM_MAXW];
  __shared__ int nlive;
  const int g = blockIdx.x, i = blockIdx.y;
  const int wf = gm_owner(a.U, g * a.SK, a.nw), wl = gm_owner(a.U, g * a.SK + a.SK - 1, a.nw);
  if (wf == wl) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // GM_EPI_LOGITS: the penalty context of the lane's row and columns, loaded first
  uint32_t fx_sw = 0u;
  GmRowEx fx_rx;
  fx_rx.n = 0;
  if (a.epi == GM_EPI_LOGITS && a.seen) {
    const int mr = 16 * i + (lane & 15);
    fx_sw = gm_seen4(a, mr, GM_COLS * g + 16 * wave + 4 * (lane >> 4));
    gm_row_ex(a, mr, fx_rx);
  }
  if (wave == 0) {
    int cnt = 0;
    for (int base = wf; base <= wl; base += 64) {
      const int x = base + lane;
      const bool ok = x <= wl && gm_begin(a.U, x, a.nw) < gm_begin(a.U, x + 1, a.nw);
      const unsigned long long m = __ballot(ok);
      if (ok) live[cnt + __popcll(m & ((1ull << lane) - 1))] = x + g;
      cnt += __popcll(m);
    }
    if (lane == 0) nlive = cnt;
  }
  __syncthreads();
  const int np = nlive;
  const int mt = (a.M + 15) / 16;
  const size_t piece = (size_t)mt * 16 * GM_COLS;
  const int m = 16 * i + (lane & 15), g4 = lane >> 4;
  const size_t off = (((size_t)i * 4 + wave) * 64 + lane) * 4;   // accumulator order
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < np; k0 += GM_PB) {
    // GM_PB pieces' loads in flight together (indices past np re-read the last, unused)
    float4 p[GM_PB];
#pragma unroll
    for (int j = 0; j < GM_PB; ++j)
      p[j] = *reinterpret_cast<const float4*>(a.part + (size_t)live[min(k0 + j, np - 1)] * piece + off);
#pragma unroll
    for (int j = 0; j < GM_PB; ++j)
      if (k0 + j < np) { s.x += p[j].x; s.y += p[j].y; s.z += p[j].z; s.w += p[j].w; }
  }
  // lane holds row m, tiled columns 4 g4 .. + 3 of n-tile 4 g + wave
  if (a.epi == GM_EPI_LOGITS) {
    __shared__ uint32_t rmx[4][16];
    uint32_t x = 0;
    if (m < a.M) {
      const int col = GM_COLS * g + 16 * wave + 4 * g4;
      const float sv[4] = {s.x, s.y, s.z, s.w};
      uint32_t b[4];
      gm_logits4(a, sv, col, fx_sw, fx_rx, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) x = max(x, gm_ord16(b[e]));
      *reinterpret_cast<uint2*>(a.C + (size_t)m * a.ldc + col) =
          make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
    }
    x = gm_rowmax_lanes(x);
    if (g4 == 0) rmx[wave][lane & 15] = x;
    __syncthreads();
    if (tid < 16) {
      const uint32_t r = max(max(rmx[0][tid], rmx[1][tid]), max(rmx[2][tid], rmx[3][tid]));
      gm_rowmax_put(a, 16 * i + tid, GM_RM_SLOTS * a.nw + wl, r);
    }
  } else if (a.epi == GM_EPI_ARGMAX) {
    const int col = GM_COLS * g + 16 * wave + 4 * g4;
    const float sv[4] = {s.x, s.y, s.z, s.w};
    uint64_t best = gm_key(sv[0], col);
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      const uint64_t k2 = gm_key(sv[j], col + j);
      best = k2 > best ? k2 : best;
    }
    best = gm_max_xor(best, 16);
    best = gm_max_xor(best, 32);
    if (g4 == 0 && m < a.M) a.am[(size_t)m * (a.N / 16) + 4 * g + wave] = best;
  } else if (a.epi == GM_EPI_SWIGLU) {
    // partner lane (g4 ^ 2) holds the up half of the same output columns
    const float o[4] = {__shfl_xor(s.x, 32, 64), __shfl_xor(s.y, 32, 64), __shfl_xor(s.z, 32, 64),
                        __shfl_xor(s.w, 32, 64)};
    const float gv[4] = {s.x, s.y, s.z, s.w};
    if (g4 < 2 && m < a.M) {
      float y[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = round_bf16(gm_silu_bf16(gv[j]) * round_bf16(o[j]));
      const int col = 8 * (4 * g + wave) + 4 * g4;
      *reinterpret_cast<uint2*>(a.C + (size_t)m * a.ldc + col) =
          make_uint2((uint32_t)f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16),
                     (uint32_t)f32_to_bf16(y[2]) | ((uint32_t)f32_to_bf16(y[3]) << 16));
    }
  } else if (m < a.M) {
    const int col = GM_COLS * g + 16 * wave + 4 * g4;
    *reinterpret_cast<uint2*>(a.C + (size_t)m * a.ldc + col) =
        make_uint2((uint32_t)f32_to_bf16(s.x) | ((uint32_t)f32_to_bf16(s.y) << 16),
                   (uint32_t)f32_to_bf16(s.z) | ((uint32_t)f32_to_bf16(s.w) << 16));
  }
}

// The argmax of each row from its (N / 16) n-tile maxima (1024 threads, four loads in
// flight per thread); the token to out[row * stride].
constexpr int GM_AF_THREADS = 1024;
__global__ __launch_bounds__(GM_AF_THREADS) void gemm_argmax_final_kernel(
    const uint64_t* __restrict__ am, int ntiles, int32_t* __restrict__ out, long long out_stride) {
  __shared__ uint64_t red[GM_AF_THREADS / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const uint64_t* rp = am + (size_t)row * ntiles;
  uint64_t b4[4] = {0, 0, 0, 0};
  for (int t = tid; t < ntiles; t += 4 * GM_AF_THREADS) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tt = t + u * GM_AF_THREADS;
      const uint64_t v = tt < ntiles ? rp[tt] : 0;
      b4[u] = v > b4[u] ? v : b4[u];
    }
  }
  uint64_t best = b4[0];
#pragma unroll
  for (int u = 1; u < 4; ++u) best = b4[u] > best ? b4[u] : best;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) best = gm_max_xor(best, m);
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    uint64_t r = red[0];
    for (int w = 1; w < GM_AF_THREADS / 64; ++w) r = red[w] > r ? red[w] : r;
    out[(size_t)row * out_stride] = (int32_t)(0xFFFFFFFFu - (uint32_t)(r & 0xFFFFFFFFu));
  }
}

// The GEMM output completed, the residual added and the row normalised, for a
// projection that feeds the decoder's residual stream (o_proj / out_proj / down, then
// modeling_qwen3_5.py:59-60): x_out = bf16(C + residual), y = RMSNorm_{1+w}(x_out); with
// no residual (the MTP fc, whose output starts the MTP layer's residual stream and is
// normalised by its input_layernorm, mtp.py:61-73) x_out = bf16(C).
// One workgroup per row; thread t owns the 8-column chunks of lollm_rmsnorm's
// chunking, and first forms each C value the way gemm_fixup_kernel does (groups
// one workgroup finished come from C, the others are the fp32 sum of their pieces in
// slot order, rounded to bf16), so the result has the same bits as lollm_gemm
// followed by lollm_rmsnorm.  Every workgroup range is non-empty (U >= nw, checked on
// the host), so the owners of a group are exactly wf .. wl.
constexpr int GM_NORM_MAXG = 128;   // N <= 8192

__global__ __launch_bounds__(RMS_THREADS) void gemm_norm_kernel(GemmArgs a,
                                                                const uint16_t* __restrict__ res,
                                                                const uint16_t* __restrict__ w,
                                                                uint16_t* __restrict__ x_out,
                                                                uint16_t* __restrict__ y,
                                                                float eps) {
  __shared__ int own[2 * GM_NORM_MAXG];
  __shared__ float red[RMS_THREADS / 64];
  const int m = blockIdx.x, tid = threadIdx.x;
  const int n8 = a.N / 8;
  const size_t piece = (size_t)((a.M + 15) / 16) * 16 * GM_COLS;
  const size_t row = (size_t)m * a.N;
  constexpr int MAXV = RMS_CHUNKS;
  // the residual and the norm weights are loaded first, with the pieces, not after the
  // sums and the reduction: one memory round trip per launch
  uint4 wv[MAXV], hv[MAXV];
#pragma unroll
  for (int ci = 0; ci < MAXV; ++ci) {
    const int c = tid + RMS_THREADS * ci;
    wv[ci] = c < n8 ? *reinterpret_cast<const uint4*>(w + 8 * c) : make_uint4(0, 0, 0, 0);
    hv[ci] = c < n8 && res ? *reinterpret_cast<const uint4*>(res + row + 8 * c) : make_uint4(0, 0, 0, 0);
  }
  for (int g = tid; g < a.G; g += RMS_THREADS) {
    own[2 * g] = gm_owner(a.U, g * a.SK, a.nw);
    own[2 * g + 1] = gm_owner(a.U, g * a.SK + a.SK - 1, a.nw);
  }
  __syncthreads();
  float v[MAXV][8];
  float ss = 0.f;
#pragma unroll
  for (int ci = 0; ci < MAXV; ++ci) {
    const int c = tid + RMS_THREADS * ci;
    if (c < n8) {
      const int g = c / 8;
      const int wf = own[2 * g], wl = own[2 * g + 1];
      float cv[8];
      if (wf == wl) {
        const uint4 u = *reinterpret_cast<const uint4*>(a.C + (size_t)m * a.ldc + 8 * c);
        const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[e] = __uint_as_float(e & 1 ? wd[e >> 1] & 0xffff0000u : wd[e >> 1] << 16);
      } else {
        // columns 8c .. 8c + 7 = columns 8 (c % 8) .. + 7 of the group's piece row m
        const size_t off0 = (size_t)m * GM_COLS + 8 * (c % 8);
        float4 s0 = make_float4(0.f, 0.f, 0.f, 0.f), s1 = s0;
        for (int x0 = wf; x0 <= wl; x0 += GM_PB) {
          // GM_PB pieces' loads in flight together (indices past wl re-read wl, unused)
          float4 p0[GM_PB], p1[GM_PB];
#pragma unroll
          for (int j = 0; j < GM_PB; ++j) {
            const float* pp = a.part + (size_t)(min(x0 + j, wl) + g) * piece + off0;
            p0[j] = *reinterpret_cast<const float4*>(pp);
            p1[j] = *reinterpret_cast<const float4*>(pp + 4);
          }
#pragma unroll
          for (int j = 0; j < GM_PB; ++j) {
            if (x0 + j <= wl) {
              s0.x += p0[j].x; s0.y += p0[j].y; s0.z += p0[j].z; s0.w += p0[j].w;
              s1.x += p1[j].x; s1.y += p1[j].y; s1.z += p1[j].z; s1.w += p1[j].w;
            }
          }
        }
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[e] = round_bf16(sv[e]);
      }
      const uint4 h = hv[ci];
      const uint32_t hd[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // no residual: x_out is the GEMM output itself (not + 0, which would turn -0 into +0)
        const float f = res ? round_bf16(cv[e] + __uint_as_float(e & 1 ? hd[e >> 1] & 0xffff0000u : hd[e >> 1] << 16))
                            : cv[e];
        v[ci][e] = f;
        ss += f * f;
      }
      uint4 o;
      o.x = f32_to_bf16(v[ci][0]) | ((uint32_t)f32_to_bf16(v[ci][1]) << 16);
      o.y = f32_to_bf16(v[ci][2]) | ((uint32_t)f32_to_bf16(v[ci][3]) << 16);
      o.z = f32_to_bf16(v[ci][4]) | ((uint32_t)f32_to_bf16(v[ci][5]) << 16);
      o.w = f32_to_bf16(v[ci][6]) | ((uint32_t)f32_to_bf16(v[ci][7]) << 16);
      *reinterpret_cast<uint4*>(x_out + row + 8 * c) = o;
    }
  }
  const float r = rms_rstd(ss, red, a.N, eps);
#pragma unroll
  for (int ci = 0; ci < MAXV; ++ci) {
    const int c = tid + RMS_THREADS * ci;
    if (c < n8) {
      const uint4 wu = wv[ci];
      const uint32_t wd[4] = {wu.x, wu.y, wu.z, wu.w};
      uint32_t od[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) od[e >> 1] = rms_out2(v[ci][e], v[ci][e + 1], r, wd[e >> 1]);
      *reinterpret_cast<uint4*>(y + row + 8 * c) = make_uint4(od[0], od[1], od[2], od[3]);
    }
  }
}

}  // namespace lollm

using namespace lollm;

static int gemm_grid(int grid) {
  if (grid > 0) return grid;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  return cus > 0 ? 2 * cus : -1;
}

static bool gemm_shape_ok(int M, int N, int K, int epi) {
  if (M <= 0 || M > 64 || N <= 0 || K <= 0) return false;
  if (N % GM_COLS || K % GM_KC) return false;
  if (epi != GM_EPI_NONE && epi != GM_EPI_SWIGLU && epi != GM_EPI_ARGMAX && epi != GM_EPI_LOGITS)
    return false;
  return true;
}

LOLLM_API int lollm_gemm_tile_weights(const void* W, void* Wt, int N, int K, int epilogue,
                                      void* stream) {
  if (!W || !Wt || N <= 0 || K <= 0 || N % GM_COLS || K % GM_KC) return LOLLM_EINVAL;
  if (epilogue != GM_EPI_NONE && epilogue != GM_EPI_SWIGLU) return LOLLM_EINVAL;
  hipLaunchKernelGGL(gemm_tile_kernel, dim3((unsigned)((size_t)(N / 16) * (K / 32))), dim3(64), 0,
                     (hipStream_t)stream, (const uint16_t*)W, (uint16_t*)Wt, N, K, epilogue);
  return launch_status();
}

// Workspace: the fp32 pieces, slot w + group, each (M rounded up to 16) x 64.
static long long gemm_ws_bytes(int M, int N, int nw) {
  return ((long long)nw + N / GM_COLS) * ((M + 15) / 16 * 16) * GM_COLS * (long long)sizeof(float);
}

LOLLM_API long long lollm_gemm_workspace_bytes(int M, int N, int K, int grid) {
  if (!gemm_shape_ok(M, N, K, GM_EPI_NONE)) return -1;
  const int nw = gemm_grid(grid);
  if (nw <= 0 || nw > GM_MAXW) return -1;
  return gemm_ws_bytes(M, N, nw);
}

// Validates the arguments common to the GEMM entry points and launches the main kernel.
// n-tiles per group of a lollm_gemm call: 6 (96 columns) when the 96-column groups divide
// evenly over the grid and the 64-column ones would not (so the call needs no merge
// launch); else 4.  A pure function of (N, grid).
static int gemm_group_tiles(int N, int nw) {
  if (N % 96 == 0 && (N / 96) % nw == 0 && (N / GM_COLS) % nw != 0) return 6;
  return 4;
}

struct GemmLogitsArgs {   // the GM_EPI_LOGITS fields of GemmArgs
  uint16_t* rmax; long long rmax_ld; const uint32_t* seen; int seen_words; const int32_t* extra;
  int extra_stride, n_extra0, T; float pen;
};

static int gemm_main(GemmArgs& a, const void* A, long long lda, const void* Wt, void* C,
                     long long ldc, int M, int N, int K, int epilogue, void* workspace,
                     long long workspace_bytes, int grid, int rowmajor, hipStream_t st,
                     bool allow_wide = false, const GemmLogitsArgs* lg = nullptr) {
  if (!A || !Wt || !C || !workspace) return LOLLM_EINVAL;
  if (!gemm_shape_ok(M, N, K, epilogue)) return LOLLM_EUNSUPPORTED;
  const long long outc = epilogue == GM_EPI_SWIGLU ? N / 2 : N;
  if (lda < K || ldc < outc || lda % 8 || ldc % 4) return LOLLM_EINVAL;
  if (grid < 0 || grid > GM_MAXW) return LOLLM_EINVAL;
  const int nw = gemm_grid(grid);
  if (nw <= 0 || nw > GM_MAXW) return LOLLM_EUNSUPPORTED;
  if (workspace_bytes < gemm_ws_bytes(M, N, nw)) return LOLLM_EINVAL;
  if ((long long)(N / GM_COLS) * (K / GM_KC) >= (1LL << 31)) return LOLLM_EUNSUPPORTED;
  a.A = (const uint16_t*)A; a.Wt = (const uint16_t*)Wt; a.C = (uint16_t*)C;
  a.part = (float*)workspace;
  a.lda = lda; a.ldc = ldc;
  const int nt = allow_wide ? gemm_group_tiles(N, nw) : 4;
  a.M = M; a.N = N; a.K = K; a.G = N / (16 * nt); a.SK = K / GM_KC; a.nw = nw; a.epi = epilogue;
  a.U = a.G * a.SK;
  a.rowmajor = rowmajor;
  a.am = nullptr;
  a.rmax = nullptr; a.rmax_ld = 0; a.seen = nullptr; a.seen_words = 0; a.extra = nullptr;
  a.extra_stride = 0; a.n_extra0 = 0; a.T = 1; a.pen = 1.f;
  if (epilogue == GM_EPI_ARGMAX)
    a.am = (uint64_t*)((char*)workspace + ((gemm_ws_bytes(M, N, nw) + 255) / 256) * 256);
  if (epilogue == GM_EPI_LOGITS) {
    if (!lg) return LOLLM_EINVAL;
    a.rmax = lg->rmax; a.rmax_ld = lg->rmax_ld; a.seen = lg->seen; a.seen_words = lg->seen_words;
    a.extra = lg->extra; a.extra_stride = lg->extra_stride; a.n_extra0 = lg->n_extra0;
    a.T = lg->T; a.pen = lg->pen;
  }
  switch ((M + 15) / 16) {
    case 1:
      if (nt == 6) hipLaunchKernelGGL((gemm_ksplit_kernel<1, 6>), dim3(nw), dim3(256), 0, st, a);
      else hipLaunchKernelGGL((gemm_ksplit_kernel<1, 4>), dim3(nw), dim3(256), 0, st, a);
      break;
    case 2:
      if (nt == 6) hipLaunchKernelGGL((gemm_ksplit_kernel<2, 6>), dim3(nw), dim3(256), 0, st, a);
      else hipLaunchKernelGGL((gemm_ksplit_kernel<2, 4>), dim3(nw), dim3(256), 0, st, a);
      break;
    default:   // 33..64 rows: the warp-specialised stream (64-row tiles, rows past M clamped)
      if (nt == 6)
        hipLaunchKernelGGL(gemm_stream_kernel<6>, dim3(nw), dim3(GS_THREADS), 0, st, a);
      else
        hipLaunchKernelGGL(gemm_stream_kernel<4>, dim3(nw), dim3(GS_THREADS), 0, st, a);
      break;
  }
  return launch_status();
}

LOLLM_API int lollm_gemm(const void* A, long long lda, const void* Wt, void* C, long long ldc,
                         int M, int N, int K, int epilogue, void* workspace,
                         long long workspace_bytes, int grid, void* stream) {
  if (epilogue != GM_EPI_NONE && epilogue != GM_EPI_SWIGLU) return LOLLM_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  GemmArgs a;
  int rc = gemm_main(a, A, lda, Wt, C, ldc, M, N, K, epilogue, workspace, workspace_bytes, grid, 0, st,
                     true);
  if (rc) return rc;
  // every range a whole number of whole groups (grid divides the groups, always so for
  // 96-column groups): nothing to merge
  if (a.G % a.nw == 0) return LOLLM_OK;
  hipLaunchKernelGGL(gemm_fixup_kernel, dim3(a.G, (M + 15) / 16), dim3(256), 0, st, a);
  return launch_status();
}

// Workspace of lollm_gemm_argmax: the pieces, then the (M, N / 16) n-tile maxima.
static long long gemm_argmax_ws_bytes(int M, int N, int nw) {
  return (gemm_ws_bytes(M, N, nw) + 255) / 256 * 256 + (long long)M * (N / 16) * 8;
}

LOLLM_API long long lollm_gemm_argmax_workspace_bytes(int M, int N, int K, int grid) {
  if (!gemm_shape_ok(M, N, K, GM_EPI_NONE)) return -1;
  const int nw = gemm_grid(grid);
  if (nw <= 0 || nw > GM_MAXW) return -1;
  return gemm_argmax_ws_bytes(M, N, nw);
}

LOLLM_API int lollm_gemm_argmax(const void* A, long long lda, const void* Wt, int M, int N, int K,
                                int32_t* out, long long out_stride, void* workspace,
                                long long workspace_bytes, int grid, void* stream) {
  if (!out || out_stride < 1) return LOLLM_EINVAL;
  if (!gemm_shape_ok(M, N, K, GM_EPI_NONE)) return LOLLM_EUNSUPPORTED;
  const int nw = gemm_grid(grid);
  if (nw <= 0 || nw > GM_MAXW) return LOLLM_EUNSUPPORTED;
  if (workspace_bytes < gemm_argmax_ws_bytes(M, N, nw)) return LOLLM_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  GemmArgs a;
  // no output matrix: the main kernel and the merge write n-tile maxima only (C is never
  // written in this epilogue; the workspace stands in for the pointer check)
  int rc = gemm_main(a, A, lda, Wt, workspace, N, M, N, K, GM_EPI_ARGMAX, workspace, workspace_bytes,
                     grid, 0, st);
  if (rc) return rc;
  if (a.G % a.nw) {
    hipLaunchKernelGGL(gemm_fixup_kernel, dim3(a.G, (M + 15) / 16), dim3(256), 0, st, a);
    rc = launch_status();
    if (rc) return rc;
  }
  hipLaunchKernelGGL(gemm_argmax_final_kernel, dim3(M), dim3(GM_AF_THREADS), 0, st,
                     (const uint64_t*)a.am, N / 16, out, out_stride);
  return launch_status();
}

LOLLM_API int lollm_gemm_rowmax_slots(int grid) {
  const int nw = gemm_grid(grid);
  if (nw <= 0 || nw > GM_MAXW) return -1;
  return (GM_RM_SLOTS + 1) * nw;
}

LOLLM_API int lollm_gemm_logits(const void* A, long long lda, const void* Wt, int M, int N, int K,
                                void* C, long long ldc, uint16_t* rowmax, long long rowmax_ld,
                                const uint32_t* seen, int seen_words, const int32_t* extra,
                                int extra_stride, int n_extra0, int T, float penalty,
                                void* workspace, long long workspace_bytes, int grid,
                                void* stream) {
  if (!rowmax) return LOLLM_EINVAL;
  const int slots = lollm_gemm_rowmax_slots(grid);
  if (slots < 0) return LOLLM_EUNSUPPORTED;
  if (rowmax_ld < slots) return LOLLM_EINVAL;
  if (seen) {
    if (T <= 0 || M % T || seen_words < (N + 31) / 32 || n_extra0 < 0) return LOLLM_EINVAL;
    if (extra && extra_stride < n_extra0 + T - 1) return LOLLM_EINVAL;
    if (extra && n_extra0 + T - 1 > GM_MAXEX) return LOLLM_EUNSUPPORTED;
    if (!(penalty > 0.f) || !(penalty < 3.0e38f)) return LOLLM_EINVAL;
  }
  GemmLogitsArgs lg{rowmax, rowmax_ld, seen, seen_words, seen ? extra : nullptr, extra_stride,
                    n_extra0, T > 0 ? T : 1, penalty};
  hipStream_t st = (hipStream_t)stream;
  GemmArgs a;
  int rc = gemm_main(a, A, lda, Wt, C, ldc, M, N, K, GM_EPI_LOGITS, workspace, workspace_bytes,
                     grid, 0, st, false, &lg);
  if (rc) return rc;
  if (a.G % a.nw == 0) return LOLLM_OK;
  hipLaunchKernelGGL(gemm_fixup_kernel, dim3(a.G, (M + 15) / 16), dim3(256), 0, st, a);
  return launch_status();
}

LOLLM_API int lollm_gemm_rmsnorm(const void* A, long long lda, const void* Wt, int M, int N, int K,
                                 const void* residual, const void* norm_w, float eps, void* C,
                                 void* x_out, void* y, void* workspace, long long workspace_bytes,
                                 int grid, void* stream) {
  if (!norm_w || !x_out || !y) return LOLLM_EINVAL;   // residual may be null
  if (N > 8 * RMS_THREADS * RMS_CHUNKS) return LOLLM_EUNSUPPORTED;
  if (M <= 0 || N <= 0 || K <= 0 || N % GM_COLS || K % GM_KC) return LOLLM_EUNSUPPORTED;
  const int nw = gemm_grid(grid);
  if (nw <= 0 || (long long)(N / GM_COLS) * (K / GM_KC) < nw) return LOLLM_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  GemmArgs a;
  int rc = gemm_main(a, A, lda, Wt, C, N, M, N, K, GM_EPI_NONE, workspace, workspace_bytes, grid, 1, st);
  if (rc) return rc;
  hipLaunchKernelGGL(gemm_norm_kernel, dim3(M), dim3(RMS_THREADS), 0, st, a, (const uint16_t*)residual,
                     (const uint16_t*)norm_w, (uint16_t*)x_out, (uint16_t*)y, eps);
  return launch_status();
}

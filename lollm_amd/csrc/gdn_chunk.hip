// Chunked Gated DeltaNet mixer for long calls (prefill), gfx950.  The layer is the one
// lollm_gdn_layer computes -- causal conv + SiLU (src/qwen3_5/blocks.py:268-286), beta /
// g gating (:313-314), L2 norm of q and k (:124-127), the delta rule, the gated
// RMSNorm (:38-51,324) -- with the delta rule in its parallel
// chunked form (torch_chunk_gated_delta_rule, blocks.py:59-113, which the reference
// runs for every T > 1 call, :316-322), and the same conv-window / state placement as
// the long-call path of gdn_layer.hip (final state in slot 0 of the half being
// written, final K-1 raw inputs in rows 0 .. K-2 of the window half being written).
//
// One 256-thread workgroup per (sequence b, v-head h) walks the chunks of 64 tokens in
// order; the 128 x 128 fp32 state S[key][value] stays in LDS.  Per chunk, with
// gc = cumsum(g), s = Dk^-0.5 and every product an fp32 MFMA (v_mfma_f32_16x16x4f32:
// the reference's fp32 arithmetic up to summation order):
//   A  = -(beta_i k_i.k_j) exp(gc_i - gc_j), j < i          (:99-100)
//   Tm = (I - A)^-1, by the reference's row recurrence (:101-103): one wave, each lane a
//        column in registers, rows broadcast with readlane
//   W  = Tm diag(beta e^gc) K,   V' = Tm diag(beta) V - W S   (:104-105, :113)
//   O  = diag(s e^gc) Q S + [s (q_i.k_j) exp(gc_i - gc_j)]_{j<=i} V'   (:112-115)
//   S <- e^gc_63 S + K^T diag(e^(gc_63 - gc)) V'              (:116-117)
// q and k enter the products as their bf16 conv outputs with the L2-norm factors
// rq_t, rk_t applied as fp32 row scales (the normalised vectors are never rounded),
// which is the arithmetic of the recurrent kernels, so a prefill and the decode steps
// after it agree.  Tokens past T in the last chunk enter with q = k = v = 0 and
// beta = g = 0 and change nothing, as the reference's zero padding (:77-80).
#include "gdn_common.h"

namespace lollm {

constexpr int GC_C = 64;     // tokens per chunk
constexpr int GC_PB = 136;   // bf16 pitch of the 64 x 128 operand tiles
constexpr int GC_PS = 132;   // fp32 pitch of the 64 x 128 matrix
constexpr int GC_PSS = 144;  // fp32 pitch of the state (conflict-free operand reads)
constexpr int GC_PT = 68;    // fp32 pitch of 64-column matrices

typedef float gc_f32x4 __attribute__((ext_vector_type(4)));

struct GcSmem {
  uint16_t kb[GC_C][GC_PB];    // k of the chunk (bf16 conv output)
  uint16_t qv[GC_C][GC_PB];    // v of the chunk, then q
  float sm[GL_DK][GC_PSS];     // the state S[key][value]
  float tm[GC_C][GC_PT];       // raw q (bf16 view) -> A -> Tm -> masked s q.k decay
  float wm[GC_C][GC_PS];       // W -> V' -> O
  float gcv[GC_C], egv[GC_C], btv[GC_C], gv[GC_C], rqv[GC_C], rkv[GC_C];
  float fwv[GC_C], f7v[GC_C];  // rk beta e^gc (W), rk e^(gc_63 - gc) (state update)
};
static_assert(sizeof(GcSmem) <= 160 * 1024, "LDS budget");

__device__ __forceinline__ float gc_bf(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

__device__ __forceinline__ gc_f32x4 gc_mma(float a, float b, gc_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256) void gdn_chunk_kernel(GdnLayerArgs a) {
  __shared__ GcSmem sh;
  uint16_t (*qraw)[GC_PB] = reinterpret_cast<uint16_t (*)[GC_PB]>(&sh.tm[0][0]);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, kq = lane >> 4;   // MFMA lane coordinates
  const int b = blockIdx.x / a.Hv, h = blockIdx.x % a.Hv;
  const int vpk = a.Hv / a.Hk, hk = h / vpk;
  const bool write_qk = (h % vpk) == 0;
  const int Km1 = a.K - 1;   // == 3 on this path
  constexpr size_t SS = (size_t)GL_DK * GL_DK;
  int off = a.conv_off[b];
  off = off < 0 ? 0 : (off > 2 * a.W - Km1 ? 2 * a.W - Km1 : off);
  const int wbase = off >= a.W ? 0 : a.W;
  int slot = a.rec_slot[b];
  slot = slot < 0 ? 0 : (slot >= 2 * a.S ? 2 * a.S - 1 : slot);
  const int rbase = slot >= a.S ? 0 : a.S;
  const size_t win_b = (size_t)b * 2 * a.W;
  const float qscale = rsqrtf((float)GL_DK);
  const float a_log = a.A_log[h], dtb = a.dt_bias[h];

  auto gchan = [&](int lc) {
    return lc < GL_DK ? hk * GL_DK + lc
                      : (lc < 2 * GL_DK ? a.key_dim + hk * GL_DK + (lc - GL_DK)
                                        : 2 * a.key_dim + h * GL_DK + (lc - 2 * GL_DK));
  };

  // ---- initial state ----
  {
    const float* s0 = a.rec + ((size_t)(b * 2 * a.S + slot) * a.Hv + h) * SS;
    for (int i = tid; i < GL_DK * GL_DK / 4; i += 256) {
      const int row = i / (GL_DK / 4), c4 = (i % (GL_DK / 4)) * 4;
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (!a.fresh) f = *reinterpret_cast<const float4*>(s0 + (size_t)row * GL_DK + c4);
      sh.sm[row][c4] = f.x; sh.sm[row][c4 + 1] = f.y; sh.sm[row][c4 + 2] = f.z; sh.sm[row][c4 + 3] = f.w;
    }
  }

  for (int t0 = 0; t0 < a.T; t0 += GC_C) {
    // ================= A. conv + SiLU =================
    // thread = (8-channel vector cv of the 48, 16-token group tg of the 4); its 19 input
    // rows (3 history + 16) are loaded as 16-byte vectors before any use
    __syncthreads();   // chunk buffers free
    if (tid < 48 * 4) {
      const int cv = tid % 48, tg = tid / 48, lc0 = cv * 8, c0 = gchan(lc0);
      const int tb = t0 + 16 * tg;            // first token of the group
      u32x4_t raw[19];
#pragma unroll
      for (int r = 0; r < 19; ++r) {
        const int t = tb - 3 + r;
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (t < 0) v = *reinterpret_cast<const u32x4_t*>(a.win + (win_b + off + 3 + t) * a.C + c0);
        else if (t < a.T) v = *reinterpret_cast<const u32x4_t*>(a.proj + ((size_t)b * a.T + t) * a.P + c0);
        raw[r] = v;
      }
      float w[8][4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint2 wv = *reinterpret_cast<const uint2*>(a.conv_w + (size_t)(c0 + e) * 4);
        w[e][0] = __uint_as_float(wv.x << 16); w[e][1] = __uint_as_float(wv.x & 0xffff0000u);
        w[e][2] = __uint_as_float(wv.y << 16); w[e][3] = __uint_as_float(wv.y & 0xffff0000u);
      }
      uint16_t* dst = cv < 16 ? &qraw[0][0] : (cv < 32 ? &sh.kb[0][0] : &sh.qv[0][0]);
      const int col = (cv % 16) * 8;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        uint32_t od[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float o2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int ee = e + u;
            float acc = 0.f;
#pragma unroll
            for (int tau = 0; tau < 4; ++tau) {
              const uint32_t wd = raw[r + tau][ee >> 1];
              acc = fmaf(w[ee][tau], __uint_as_float(ee & 1 ? wd & 0xffff0000u : wd << 16), acc);
            }
            o2[u] = tb + r < a.T ? round_bf16(silu_g(round_bf16(acc))) : 0.f;
          }
          od[e >> 1] = f32_to_bf16(o2[0]) | ((uint32_t)f32_to_bf16(o2[1]) << 16);
        }
        *reinterpret_cast<u32x4_t*>(dst + (16 * tg + r) * GC_PB + col) = u32x4_t{od[0], od[1], od[2], od[3]};
      }
    }
    if (tid < GC_C) {
      const int t = t0 + tid;
      float gg = 0.f, bb = 0.f;
      if (t < a.T) {
        const size_t base = ((size_t)b * a.T + t) * a.P + a.C + a.value_dim;
        const float braw = gc_bf(a.proj[base + h]);
        const float araw = gc_bf(a.proj[base + a.Hv + h]);
        gg = -__expf(a_log) * softplus_g(araw + dtb);
        bb = round_bf16(1.f / (1.f + __expf(-braw)));
      }
      sh.gv[tid] = gg;
      sh.btv[tid] = bb;
    }
    __syncthreads();
    // L2-norm factors of q and k per token (4 threads x 32 channels); q stays in
    // registers until V is consumed
    uint32_t qreg[16];
    {
      const int tok = tid >> 2, part = tid & 3;
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int e = 0; e < 32; e += 2) {
        const uint16_t q0 = qraw[tok][part * 32 + e], q1 = qraw[tok][part * 32 + e + 1];
        const float xq0 = gc_bf(q0), xq1 = gc_bf(q1);
        const float xk0 = gc_bf(sh.kb[tok][part * 32 + e]), xk1 = gc_bf(sh.kb[tok][part * 32 + e + 1]);
        sq = fmaf(xq0, xq0, sq); sq = fmaf(xq1, xq1, sq);
        sk = fmaf(xk0, xk0, sk); sk = fmaf(xk1, xk1, sk);
        qreg[e / 2] = (uint32_t)q0 | ((uint32_t)q1 << 16);
      }
      sq += __shfl_xor(sq, 1, 64); sq += __shfl_xor(sq, 2, 64);
      sk += __shfl_xor(sk, 1, 64); sk += __shfl_xor(sk, 2, 64);
      if (part == 0) {
        sh.rqv[tok] = rsqrtf(sq + 1e-6f);
        sh.rkv[tok] = rsqrtf(sk + 1e-6f);
      }
    }
    if (tid == 0) {
      float run = 0.f;
      for (int i = 0; i < GC_C; ++i) {
        run += sh.gv[i];
        sh.gcv[i] = run;
      }
    }
    __syncthreads();
    if (tid < GC_C) {
      const float eg = expf(sh.gcv[tid]);
      sh.egv[tid] = eg;
      sh.fwv[tid] = sh.rkv[tid] * sh.btv[tid] * eg;
      sh.f7v[tid] = sh.rkv[tid] * expf(sh.gcv[GC_C - 1] - sh.gcv[tid]);
    }
    // ================= B1. A = -(beta_i k_i.k_j) exp(gc_i - gc_j), j < i =================
    {
      const int ti = wave;
      gc_f32x4 acc[4];
#pragma unroll
      for (int tj = 0; tj < 4; ++tj) acc[tj] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int k0 = 0; k0 < GL_DK; k0 += 4) {
        const float av = gc_bf(sh.kb[16 * ti + r16][k0 + kq]);
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
          if (tj <= ti) acc[tj] = gc_mma(av, gc_bf(sh.kb[16 * tj + r16][k0 + kq]), acc[tj]);
      }
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 16 * ti + 4 * kq + j, jj = 16 * tj + r16;
          sh.tm[i][jj] = jj < i ? -sh.btv[i] * (acc[tj][j] * sh.rkv[i] * sh.rkv[jj]) * expf(sh.gcv[i] - sh.gcv[jj]) : 0.f;
        }
    }
    __syncthreads();
    // ================= B2. Tm = (I - A)^-1 (wave 0) =================
    if (wave == 0) {
      // lane j holds column j; row i's original entries (still in LDS until the end)
      // are read as broadcasts, four at a time
      float col[GC_C];
#pragma unroll
      for (int m = 0; m < GC_C; ++m) col[m] = sh.tm[m][lane];
#pragma unroll
      for (int i = 1; i < GC_C; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int m4 = 0; m4 < i; m4 += 4) {
          const float4 rowv = *reinterpret_cast<const float4*>(&sh.tm[i][m4]);
          const float rv[4] = {rowv.x, rowv.y, rowv.z, rowv.w};
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (m4 + u < i) acc = fmaf(rv[u], col[m4 + u], acc);
        }
        col[i] += acc;
      }
#pragma unroll
      for (int m = 0; m < GC_C; ++m) sh.tm[m][lane] = col[m] + (m == lane ? 1.f : 0.f);
    }
    __syncthreads();
    // ================= B3/B4. W and V' for this wave's 16 rows =================
    // k outer, the 8 column tiles inner: each a operand is loaded once per k step
    const int rw = 16 * wave;          // first row of this wave's row tile
    const int nkb = wave + 1;          // 16-wide k blocks below the diagonal (Tm is lower triangular)
    gc_f32x4 vn[8];
    {
      gc_f32x4 acc[8];
#pragma unroll
      for (int tc = 0; tc < 8; ++tc) acc[tc] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
      for (int kb16 = 0; kb16 < nkb; ++kb16) {
#pragma unroll
        for (int k4 = 0; k4 < 16; k4 += 4) {
          const int kk = 16 * kb16 + k4 + kq;
          const float av = sh.tm[rw + r16][kk], f = sh.fwv[kk];
#pragma unroll
          for (int tc = 0; tc < 8; ++tc) acc[tc] = gc_mma(av, gc_bf(sh.kb[kk][16 * tc + r16]) * f, acc[tc]);
        }
      }
#pragma unroll
      for (int tc = 0; tc < 8; ++tc)
#pragma unroll
        for (int j = 0; j < 4; ++j) sh.wm[rw + 4 * kq + j][16 * tc + r16] = acc[tc][j];
      // V' = Tm diag(beta) V - W S, one accumulator per tile (W S enters with -S)
#pragma unroll
      for (int tc = 0; tc < 8; ++tc) vn[tc] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
      for (int kb16 = 0; kb16 < nkb; ++kb16) {
#pragma unroll
        for (int k4 = 0; k4 < 16; k4 += 4) {
          const int kk = 16 * kb16 + k4 + kq;
          const float av = sh.tm[rw + r16][kk], f = sh.btv[kk];
#pragma unroll
          for (int tc = 0; tc < 8; ++tc) vn[tc] = gc_mma(av, gc_bf(sh.qv[kk][16 * tc + r16]) * f, vn[tc]);
        }
      }
#pragma unroll 4
      for (int k0 = 0; k0 < GL_DK; k0 += 4) {
        const float av = sh.wm[rw + r16][k0 + kq];
#pragma unroll
        for (int tc = 0; tc < 8; ++tc) vn[tc] = gc_mma(av, -sh.sm[k0 + kq][16 * tc + r16], vn[tc]);
      }
    }
    __syncthreads();   // every wave done with V (qv) and W
#pragma unroll
    for (int tc = 0; tc < 8; ++tc)
#pragma unroll
      for (int j = 0; j < 4; ++j) sh.wm[rw + 4 * kq + j][16 * tc + r16] = vn[tc][j];
    {
      const int tok = tid >> 2, part = tid & 3;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sh.qv[tok][part * 32 + 2 * e] = (uint16_t)(qreg[e] & 0xffffu);
        sh.qv[tok][part * 32 + 2 * e + 1] = (uint16_t)(qreg[e] >> 16);
      }
    }
    __syncthreads();
    // ================= B5. masked s q.k decay (this wave's rows) =================
    {
      gc_f32x4 acc[4];
#pragma unroll
      for (int tj = 0; tj < 4; ++tj) acc[tj] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int k0 = 0; k0 < GL_DK; k0 += 4) {
        const float av = gc_bf(sh.qv[rw + r16][k0 + kq]);
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
          if (tj <= wave) acc[tj] = gc_mma(av, gc_bf(sh.kb[16 * tj + r16][k0 + kq]), acc[tj]);
      }
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = rw + 4 * kq + j, jj = 16 * tj + r16;
          sh.tm[i][jj] = jj <= i ? (acc[tj][j] * sh.rqv[i] * sh.rkv[jj]) * qscale * expf(sh.gcv[i] - sh.gcv[jj]) : 0.f;
        }
    }
    // ================= B6. O = diag(s e^gc) Q S + intra V' =================
    // the row scale rq s e^gc rides on the a operand (one row per lane)
    gc_f32x4 ov[8];
    {
      const int ir = rw + r16;
      const float rs = sh.rqv[ir] * qscale * sh.egv[ir];
#pragma unroll
      for (int tc = 0; tc < 8; ++tc) ov[tc] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int k0 = 0; k0 < GL_DK; k0 += 4) {
        const float av = gc_bf(sh.qv[ir][k0 + kq]) * rs;
#pragma unroll
        for (int tc = 0; tc < 8; ++tc) ov[tc] = gc_mma(av, sh.sm[k0 + kq][16 * tc + r16], ov[tc]);
      }
      for (int kb16 = 0; kb16 < nkb; ++kb16) {
#pragma unroll
        for (int k4 = 0; k4 < 16; k4 += 4) {
          const int kk = 16 * kb16 + k4 + kq;
          const float av = sh.tm[ir][kk];
#pragma unroll
          for (int tc = 0; tc < 8; ++tc) ov[tc] = gc_mma(av, sh.wm[kk][16 * tc + r16], ov[tc]);
        }
      }
    }
    __syncthreads();   // every wave done reading S
    // ================= B7. S <- e^gc_63 S + K^T diag(e^(gc_63 - gc)) V' =================
    // this wave's 32 key rows x 128 value columns: 2 x 8 tiles, t outer
    {
      const float elast = sh.egv[GC_C - 1];
      gc_f32x4 acc[2][8];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int tc = 0; tc < 8; ++tc) acc[u][tc] = gc_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
      for (int k0 = 0; k0 < GC_C; k0 += 4) {
        const int t = k0 + kq;
        const float f = sh.f7v[t];
        const float a0 = gc_bf(sh.kb[t][32 * wave + r16]), a1 = gc_bf(sh.kb[t][32 * wave + 16 + r16]);
#pragma unroll
        for (int tc = 0; tc < 8; ++tc) {
          const float bv = sh.wm[t][16 * tc + r16] * f;
          acc[0][tc] = gc_mma(a0, bv, acc[0][tc]);
          acc[1][tc] = gc_mma(a1, bv, acc[1][tc]);
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int tc = 0; tc < 8; ++tc)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float& sv = sh.sm[32 * wave + 16 * u + 4 * kq + j][16 * tc + r16];
            sv = fmaf(elast, sv, acc[u][tc][j]);
          }
    }
    __syncthreads();   // every wave done reading V'
#pragma unroll
    for (int tc = 0; tc < 8; ++tc)
#pragma unroll
      for (int j = 0; j < 4; ++j) sh.wm[rw + 4 * kq + j][16 * tc + r16] = ov[tc][j];
    __syncthreads();
    // ================= B8. gated RMSNorm, 16 threads per token, 8 columns each =================
    for (int tb = 0; tb < GC_C; tb += 16) {
      const int i = tb + (tid >> 4), part = tid & 15, t = t0 + i;
      float ovs[8], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ovs[e] = round_bf16(sh.wm[i][part * 8 + e]);   // the core output is a bf16 tensor
        ss += ovs[e] * ovs[e];
      }
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, 64);
      if (t < a.T) {
        const float rr = rsqrtf(ss / (float)GL_DK + a.eps);
        const size_t zb = ((size_t)b * a.T + t) * a.P + a.C + (size_t)h * GL_DK + part * 8;
        const uint4 zu = *reinterpret_cast<const uint4*>(a.proj + zb);
        const uint4 wu = *reinterpret_cast<const uint4*>(a.norm_w + part * 8);
        const uint32_t zd[4] = {zu.x, zu.y, zu.z, zu.w}, wd[4] = {wu.x, wu.y, wu.z, wu.w};
        uint32_t od[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float y2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int ee = e + u;
            const float z = __uint_as_float(ee & 1 ? zd[ee >> 1] & 0xffff0000u : zd[ee >> 1] << 16);
            const float w = __uint_as_float(ee & 1 ? wd[ee >> 1] & 0xffff0000u : wd[ee >> 1] << 16);
            const float hn = round_bf16(ovs[ee] * rr);
            y2[u] = round_bf16(w * hn) * silu_g(z);
          }
          od[e >> 1] = f32_to_bf16(y2[0]) | ((uint32_t)f32_to_bf16(y2[1]) << 16);
        }
        *reinterpret_cast<uint4*>(a.out + ((size_t)b * a.T + t) * a.value_dim + (size_t)h * GL_DK +
                                  part * 8) = make_uint4(od[0], od[1], od[2], od[3]);
      }
    }
  }
  __syncthreads();
  // ---- final state in slot 0 of the written half; final K-1 raw inputs in the window ----
  {
    float* sf = a.rec + ((size_t)(b * 2 * a.S + rbase) * a.Hv + h) * SS;
    for (int i = tid; i < GL_DK * GL_DK / 4; i += 256) {
      const int row = i / (GL_DK / 4), c4 = (i % (GL_DK / 4)) * 4;
      *reinterpret_cast<float4*>(sf + (size_t)row * GL_DK + c4) =
          make_float4(sh.sm[row][c4], sh.sm[row][c4 + 1], sh.sm[row][c4 + 2], sh.sm[row][c4 + 3]);
    }
    for (int i = tid; i < Km1 * GL_CH; i += 256) {
      const int r = i / GL_CH, lc = i % GL_CH;
      if (lc >= 2 * GL_DK || write_qk) {
        const int c = gchan(lc);
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
                                      const int32_t* rec_slot, int slots, int fresh, void* out,
                                      int B, int T, int Hk, int Hv, int Dk, int Dv, int conv_kernel,
                                      float eps, void* stream) {
  if (!proj || !conv_w || !A_log || !dt_bias || !norm_w || !win || !conv_off || !rec ||
      !rec_slot || !out)
    return LOLLM_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return LOLLM_EINVAL;
  if (Dk != GL_DK || Dv != GL_DK || conv_kernel != 4) return LOLLM_EUNSUPPORTED;
  if (win_rows < conv_kernel - 1 || slots < 1) return LOLLM_EINVAL;
  // the long-call placement: no per-position snapshots, the window half too short to
  // hold the whole call (so only the final K-1 raw rows are written)
  if (T <= slots || conv_kernel - 1 + T <= win_rows || T < conv_kernel - 1) return LOLLM_EUNSUPPORTED;
  const int key_dim = Hk * Dk, value_dim = Hv * Dv, C = 2 * key_dim + value_dim;
  if (proj_stride < (long long)C + value_dim + 2 * Hv || proj_stride % 8) return LOLLM_EINVAL;
  GdnLayerArgs a;
  a.proj = (const uint16_t*)proj; a.conv_w = (const uint16_t*)conv_w; a.A_log = A_log;
  a.dt_bias = dt_bias; a.norm_w = (const uint16_t*)norm_w; a.win = (uint16_t*)win;
  a.conv_off = conv_off; a.rec = rec; a.rec_slot = rec_slot; a.out = (uint16_t*)out;
  a.P = proj_stride; a.T = T; a.Hk = Hk; a.Hv = Hv; a.C = C; a.key_dim = key_dim;
  a.value_dim = value_dim; a.K = conv_kernel; a.W = win_rows; a.S = slots; a.fresh = fresh ? 1 : 0;
  a.eps = eps;
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(B * Hv), dim3(256), 0, (hipStream_t)stream, a);
  return launch_status();
}

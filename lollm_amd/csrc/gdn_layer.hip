// The Gated DeltaNet mixer of one decoder layer, fused from the in_proj outputs to the
// gated-norm output (gfx950).  Reference: GatedDeltaNet.forward, src/qwen3_5/blocks.py
// :288-329, i.e. steps 2-6 below; the projections before and out_proj after are GEMMs.
//
// Per (sequence b, v-head h) workgroup of 256 threads, tokens in chunks of GL_TC:
//   1. causal depthwise conv (kernel K, no bias) over [conv state | raw x] for the
//      384 channels this head reads (q and k of qk-head h / v_per_k, v of head h),
//      then SiLU (blocks.py:268-286; the new conv state is the last K-1 RAW inputs);
//   2. beta = sigmoid(b) in bf16, g = -exp(A_log) softplus(a + dt_bias) in fp32
//      (blocks.py:313-314);
//   3. the recurrent delta rule with in-kernel L2 norm of q, k and q scaled by
//      Dk^-0.5 (blocks.py:116-144), the 128 x 128 fp32 state held in registers exactly
//      as in gdn_verify.hip (wave = 32-column slab, lane = 16 rows x 4 columns);
//   4. the gated RMSNorm per v-head (blocks.py:38-51,324) and the bf16 output row.
// State lives in ping-pong buffers selected per sequence on the device: the conv
// window buffer has two halves of W rows, the recurrent state two halves, each with a
// replay record of up to S positions.  A call reads the half holding the committed
// state (conv_off[b], rec_half[b]) and writes the other one.  A short call (T <= S,
// verify / decode) first rebuilds the committed state -- the half's state plus its
// first replay[b] records -- writes it to the other half, runs its T positions and
// records them there instead of storing T states; accepting `a` drafts then only sets
// new indices (other half, replay = a + 1) and no host-side state changes between
// steps.  Nothing in the committed half is written, so a call that is not committed
// can simply be run again.
#include "gdn_common.h"

namespace lollm {

// SHORT: T <= S, the call rebuilds the committed state and records its positions
// (verify / decode); otherwise it is a long call (prefill) that starts from the state in
// the written half (lollm_gdn_layer rebuilds it there first) and stores its final state.
template <bool SHORT>
__global__ __launch_bounds__(256) void gdn_layer_kernel(GdnLayerArgs a) {
  __shared__ float xin[GL_KMAX - 1 + GL_TC][GL_CH];  // conv inputs (state rows first)
  __shared__ float act[GL_TC][GL_CH];                // q | k | v after conv + SiLU
  __shared__ float obuf[GL_TC][GL_DK];               // scan outputs
  __shared__ float gb[GL_TC][2];                     // g, beta
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = lane & 7, rg = lane >> 3;
  const int b = blockIdx.x / a.Hv, h = blockIdx.x % a.Hv;
  const int vpk = a.Hv / a.Hk, hk = h / vpk;
  const bool write_qk = (h % vpk) == 0;  // q/k window channels are shared by vpk heads
  const int row0 = rg * 16, col0 = wave * 32 + cg * 4;
  const int Km1 = a.K - 1;
  const bool full_window = Km1 + a.T <= a.W;
  constexpr size_t SS = (size_t)GL_DK * GL_DK;
  int off = a.conv_off[b];
  off = off < 0 ? 0 : (off > 2 * a.W - Km1 ? 2 * a.W - Km1 : off);  // never out of range
  const int wbase = off >= a.W ? 0 : a.W;          // window half written by this call
  const int half = a.rec_half[b] & 1, other = half ^ 1;
  int n = a.fresh ? 0 : a.replay[b];
  n = n < 0 ? 0 : (n > a.S ? a.S : n);
  float* st_out = a.rec + ((size_t)(b * 2 + other) * a.Hv + h) * SS;
  const float* st_in = SHORT ? a.rec + ((size_t)(b * 2 + half) * a.Hv + h) * SS : st_out;
  const uint8_t* rep_in = a.rep + ((size_t)(b * 2 + half) * a.Hv + h) * a.S * GL_REC_BYTES;
  uint8_t* rep_out = a.rep + ((size_t)(b * 2 + other) * a.Hv + h) * a.S * GL_REC_BYTES;
  const size_t win_b = (size_t)b * 2 * a.W;

  auto gchan = [&](int lc) {  // local channel -> global conv channel
    return lc < GL_DK ? hk * GL_DK + lc
                      : (lc < 2 * GL_DK ? a.key_dim + hk * GL_DK + (lc - GL_DK)
                                        : 2 * a.key_dim + h * GL_DK + (lc - 2 * GL_DK));
  };
  auto owns = [&](int lc) { return lc >= 2 * GL_DK || write_qk; };

  // ---- initial conv state ----
  for (int i = tid; i < Km1 * GL_CH; i += 256) {
    const int r = i / GL_CH, lc = i % GL_CH, c = gchan(lc);
    const uint16_t v = a.win[(win_b + off + r) * a.C + c];
    xin[r][lc] = bf16_to_f32(v);
    if (full_window && owns(lc)) a.win[(win_b + wbase + r) * a.C + c] = v;
  }
  // ---- recurrent state ----
  float S[16][4];
  if (!a.fresh) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float4 f = *reinterpret_cast<const float4*>(st_in + (size_t)(row0 + r) * GL_DK + col0);
      S[r][0] = f.x; S[r][1] = f.y; S[r][2] = f.z; S[r][3] = f.w;
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) S[r][0] = S[r][1] = S[r][2] = S[r][3] = 0.f;
  }
  if (SHORT) {  // the committed state: replay the accepted records, store it to the other half
    for (int j = 0; j < n; ++j) gdn_replay_one(S, rep_in + (size_t)j * GL_REC_BYTES, row0, col0);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      store_nt(st_out + (size_t)(row0 + r) * GL_DK + col0,
               make_uint4(__float_as_uint(S[r][0]), __float_as_uint(S[r][1]),
                          __float_as_uint(S[r][2]), __float_as_uint(S[r][3])));
  }
  const float a_log = a.A_log[h], dtb = a.dt_bias[h];
  const float qscale = rsqrtf((float)GL_DK);

  for (int t0 = 0; t0 < a.T; t0 += GL_TC) {
    const int tc = min(GL_TC, a.T - t0);
    __syncthreads();  // previous chunk fully consumed
    // 1a. raw inputs of this chunk (+ window copy)
    for (int i = tid; i < tc * GL_CH; i += 256) {
      const int r = i / GL_CH, lc = i % GL_CH, c = gchan(lc);
      const uint16_t v = a.proj[((size_t)b * a.T + t0 + r) * a.P + c];
      xin[Km1 + r][lc] = bf16_to_f32(v);
      if (full_window && owns(lc)) a.win[(win_b + wbase + Km1 + t0 + r) * a.C + c] = v;
    }
    if (tid < tc) {
      const size_t base = ((size_t)b * a.T + t0 + tid) * a.P + a.C + a.value_dim;
      const float bb = bf16_to_f32(a.proj[base + h]);
      const float aa = bf16_to_f32(a.proj[base + a.Hv + h]);
      gb[tid][0] = -__expf(a_log) * softplus_g(aa + dtb);
      gb[tid][1] = round_bf16(1.f / (1.f + __expf(-bb)));
    }
    __syncthreads();
    // 1b. conv + SiLU (bf16 rounding at the conv output and at the SiLU output)
    for (int i = tid; i < tc * GL_CH; i += 256) {
      const int r = i / GL_CH, lc = i % GL_CH, c = gchan(lc);
      float acc = 0.f;
      for (int tau = 0; tau < a.K; ++tau)
        acc = fmaf(bf16_to_f32(a.conv_w[(size_t)c * a.K + tau]), xin[r + tau][lc], acc);
      act[r][lc] = round_bf16(silu_g(round_bf16(acc)));
    }
    __syncthreads();
    if (SHORT)  // k | v of the chunk's records
      for (int i = tid; i < tc * 32; i += 256)
        store_nt(rep_out + (size_t)(t0 + i / 32) * GL_REC_BYTES + (i % 32) * 16,
                 gdn_record_kv(&act[i / 32][GL_DK], i % 32));
    // carry the last K-1 raw inputs as the next chunk's state
    {
      float keep[(GL_KMAX - 1) * GL_CH / 256 + 1];
      int n = 0;
      for (int i = tid; i < Km1 * GL_CH; i += 256) keep[n++] = xin[tc + i / GL_CH][i % GL_CH];
      __syncthreads();
      n = 0;
      for (int i = tid; i < Km1 * GL_CH; i += 256) xin[i / GL_CH][i % GL_CH] = keep[n++];
    }
    // 2. the scan over the chunk
    for (int i = 0; i < tc; ++i) {
      const int t = t0 + i;
      float kr[16], qr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        qr[r] = act[i][row0 + r];
        kr[r] = act[i][GL_DK + row0 + r];
      }
      float pa[4] = {0.f, 0.f, 0.f, 0.f}, pb[4] = {0.f, 0.f, 0.f, 0.f};
      float pkq = 0.f, pkk = 0.f, pqq = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          pa[c] = fmaf(S[r][c], kr[r], pa[c]);
          pb[c] = fmaf(S[r][c], qr[r], pb[c]);
        }
        pkq = fmaf(kr[r], qr[r], pkq);
        pkk = fmaf(kr[r], kr[r], pkk);
        pqq = fmaf(qr[r], qr[r], pqq);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pa[c] = sum_lanes8(pa[c]);
        pb[c] = sum_lanes8(pb[c]);
      }
      pkq = sum_lanes8(pkq);
      pkk = sum_lanes8(pkk);
      pqq = sum_lanes8(pqq);
      const float rk = rsqrtf(pkk + 1e-6f);
      const float rq = rsqrtf(pqq + 1e-6f) * qscale;
      const float kq = pkq * rk * rq;
      const float gam = __expf(gb[i][0]), bet = gb[i][1];
      float vv[4], d[4], o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) vv[c] = act[i][2 * GL_DK + col0 + c];
      gdn_delta(d, pa, vv, gam, rk, bet);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = gam * pb[c] * rq + d[c] * kq;
      if (rg == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) obuf[i][col0 + c] = o[c];
      }
      if (SHORT && tid == 0)
        store_nt(rep_out + (size_t)t * GL_REC_BYTES + 4 * GL_DK,
                 make_uint4(__float_as_uint(gam), __float_as_uint(bet), __float_as_uint(rk), 0u));
      gdn_update(S, kr, rk, d, gam);
    }
    __syncthreads();
    // 3. gated RMSNorm of each token's 128 outputs: 16 threads per token, 8 columns each
    {
      const int i = tid >> 4, part = tid & 15;
      float ov[8], ss = 0.f;
      if (i < tc) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ov[e] = round_bf16(obuf[i][part * 8 + e]);  // core output is a bf16 tensor
          ss += ov[e] * ov[e];
        }
      }
      ss = sum_lanes16(ss);
      if (i < tc) {
        const float r = rsqrtf(ss / (float)GL_DK + a.eps);
        const size_t zb = ((size_t)b * a.T + t0 + i) * a.P + a.C + (size_t)h * GL_DK + part * 8;
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
            const float hn = round_bf16(ov[ee] * r);
            y2[u] = round_bf16(w * hn) * silu_g(z);
          }
          od[e >> 1] = f32_to_bf16(y2[0]) | ((uint32_t)f32_to_bf16(y2[1]) << 16);
        }
        *reinterpret_cast<uint4*>(a.out + ((size_t)b * a.T + t0 + i) * a.value_dim +
                                  (size_t)h * GL_DK + part * 8) = make_uint4(od[0], od[1], od[2], od[3]);
      }
    }
  }
  // ---- long calls: the final state and the final conv state in rows [0, K-1) ----
  if (!SHORT) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      *reinterpret_cast<float4*>(st_out + (size_t)(row0 + r) * GL_DK + col0) =
          make_float4(S[r][0], S[r][1], S[r][2], S[r][3]);
  }
  if (!full_window) {
    __syncthreads();
    for (int i = tid; i < Km1 * GL_CH; i += 256) {
      const int r = i / GL_CH, lc = i % GL_CH;
      if (owns(lc)) a.win[(win_b + wbase + r) * a.C + gchan(lc)] = f32_to_bf16(xin[r][lc]);
    }
  }
}


// ---------------------------------------------------------------------------------
// Verify / decode form (T <= S <= GL_TC, conv kernel 4, the new window fits one half):
// the same math as gdn_layer_kernel<true>, laid out so that a workgroup makes ONE round
// trip to memory.  Every input -- the recurrent state (registers), the replay records
// (LDS), the conv window and the T projection rows of its 384 channels, the conv
// weights, z, the norm weight, b and a -- is requested in one batch before the first
// barrier; after it the workgroup only computes and stores: the rebuilt state and the
// new records stream out with non-temporal stores and no barrier ever waits for them
// (barriers order LDS only).
constexpr int GV_K = 4;

__global__ __launch_bounds__(256) void gdn_layer_verify_kernel(GdnLayerArgs a) {
  __shared__ __attribute__((aligned(16))) float xin[GV_K - 1 + GL_TC][GL_CH];  // [state | raw]
  __shared__ __attribute__((aligned(16))) float act[GL_TC][GL_CH];   // q | k | v, conv + SiLU
  __shared__ __attribute__((aligned(16))) float obuf[GL_TC][GL_DK];  // scan outputs
  __shared__ __attribute__((aligned(16))) uint16_t cw[GL_CH][GV_K];  // conv weights, 384 channels
  __shared__ __attribute__((aligned(16))) uint16_t zb[GL_TC][GL_DK]; // z rows of this head
  __shared__ __attribute__((aligned(16))) uint16_t nw[GL_DK];        // gated-norm weight
  __shared__ float gb[GL_TC][2];                                     // g, beta
  __shared__ __attribute__((aligned(16))) uint4 rbuf[GL_TC * GL_REC_U4]; // records to replay
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = lane & 7, rg = lane >> 3;
  const int b = blockIdx.x / a.Hv, h = blockIdx.x % a.Hv;
  const int vpk = a.Hv / a.Hk, hk = h / vpk;
  const bool write_qk = (h % vpk) == 0;  // q/k window channels are shared by vpk heads
  const int row0 = rg * 16, col0 = wave * 32 + cg * 4;
  const int T = a.T;
  constexpr int Km1 = GV_K - 1;
  constexpr size_t SS = (size_t)GL_DK * GL_DK;
  int off = a.conv_off[b];
  off = off < 0 ? 0 : (off > 2 * a.W - Km1 ? 2 * a.W - Km1 : off);  // never out of range
  const int wbase = off >= a.W ? 0 : a.W;          // window half written by this call
  const int half = a.rec_half[b] & 1, other = half ^ 1;
  int n = a.fresh ? 0 : a.replay[b];
  n = n < 0 ? 0 : (n > a.S ? a.S : n);             // records to replay (a.S <= GL_TC)
  const size_t hin = (size_t)(b * 2 + half) * a.Hv + h, hout = (size_t)(b * 2 + other) * a.Hv + h;
  const size_t win_b = (size_t)b * 2 * a.W;
  // channel group gi (q, k, v) -> first global conv channel
  auto gbase = [&](int gi) {
    return gi == 0 ? hk * GL_DK : (gi == 1 ? a.key_dim + hk * GL_DK : 2 * a.key_dim + h * GL_DK);
  };

  // ---- 1. one batch of loads ----
  // conv inputs: (K-1+T) rows x 3 groups x 16 chunks of 8 channels
  const int nx = (Km1 + T) * 48;
  uint4 xv[3];
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const int id = it * 256 + tid;
    xv[it] = make_uint4(0, 0, 0, 0);
    if (id < nx) {
      const int r = id / 48, gi = (id / 16) % 3, part = id % 16;
      const int c = gbase(gi) + part * 8;
      const uint16_t* src = r < Km1 ? a.win + (win_b + off + r) * a.C + c
                                    : a.proj + ((size_t)b * T + r - Km1) * a.P + c;
      xv[it] = *reinterpret_cast<const uint4*>(src);
    }
  }
  uint4 cwv = make_uint4(0, 0, 0, 0), zv = make_uint4(0, 0, 0, 0), nwv = make_uint4(0, 0, 0, 0);
  if (tid < 192) {  // 3 groups x 128 channels x 4 taps = 192 chunks of 16 B
    const int gi = tid / 64, part = tid % 64;
    cwv = *reinterpret_cast<const uint4*>(a.conv_w + (size_t)gbase(gi) * GV_K + part * 8);
  }
  if (tid < T * 16) {
    const int t = tid / 16, part = tid % 16;
    zv = *reinterpret_cast<const uint4*>(a.proj + ((size_t)b * T + t) * a.P + a.C +
                                         (size_t)h * GL_DK + part * 8);
  }
  if (tid >= 240) nwv = *reinterpret_cast<const uint4*>(a.norm_w + (tid - 240) * 8);
  // b, a of position min(tid, T - 1): unconditional, so no branch holds a wait that
  // the compiler could hoist above the state loads below (used only for tid < T)
  const size_t base_ba = ((size_t)b * T + (tid < T ? tid : T - 1)) * a.P + a.C + a.value_dim;
  const uint16_t bb_raw = a.proj[base_ba + h], aa_raw = a.proj[base_ba + a.Hv + h];
  const float a_log = a.A_log[h], dtb = a.dt_bias[h];
  // the n records to replay, 33 chunks of 16 B each (n * 33 <= 264 chunks: two per thread;
  // the descriptor ends at the n-th record, so the rest read zero and touch no memory)
  uint4 rv[2];
  {
    const __amdgpu_buffer_rsrc_t rr =
        buf_rsrc(a.rep + hin * a.S * GL_REC_BYTES, (uint32_t)(n * GL_REC_BYTES));
#pragma unroll
    for (int it = 0; it < 2; ++it)
      rv[it] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)((it * 256 + tid) * 16), 0, 2));
  }
  // The state last: every load above is waited for before the conv, and the waits are
  // in issue order, so the state (64 KB per workgroup) stays in flight through the conv,
  // gating and norms.  Its loads are unconditional -- a fresh call reads through an empty
  // descriptor (zeros, no memory touched) -- so the compiler counts them exactly.  Read
  // once per launch (a snapshot of the previous step): non-temporal.
  float S[16][4];
  {
    const float* s0 = a.rec + hin * SS;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(s0, a.fresh ? 0u : (uint32_t)(SS * sizeof(float)));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const u32x4_t f = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(((row0 + r) * GL_DK + col0) * 4), 0, 2));
      S[r][0] = __uint_as_float(f.x); S[r][1] = __uint_as_float(f.y);
      S[r][2] = __uint_as_float(f.z); S[r][3] = __uint_as_float(f.w);
    }
  }
  __builtin_amdgcn_sched_barrier(0);   // nothing that waits on a load moves above the state loads

  // ---- 2. to LDS, and the new conv window (state rows + raw inputs) to the other half ----
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const int id = it * 256 + tid;
    if (id < nx) {
      const int r = id / 48, gi = (id / 16) % 3, part = id % 16;
      const uint32_t wd[4] = {xv[it].x, xv[it].y, xv[it].z, xv[it].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xin[r][gi * GL_DK + part * 8 + 2 * e] = __uint_as_float(wd[e] << 16);
        xin[r][gi * GL_DK + part * 8 + 2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
      }
      if (gi == 2 || write_qk)
        *reinterpret_cast<uint4*>(a.win + (win_b + wbase + r) * a.C + gbase(gi) + part * 8) = xv[it];
    }
  }
  if (tid < 192) *reinterpret_cast<uint4*>(&cw[(tid / 64) * GL_DK + (tid % 64) * 2][0]) = cwv;
  if (tid < T * 16) *reinterpret_cast<uint4*>(&zb[tid / 16][(tid % 16) * 8]) = zv;
  if (tid >= 240) *reinterpret_cast<uint4*>(&nw[(tid - 240) * 8]) = nwv;
#pragma unroll
  for (int it = 0; it < 2; ++it)
    if (it * 256 + tid < GL_TC * GL_REC_U4) rbuf[it * 256 + tid] = rv[it];
  if (tid < T) {
    const float bb = bf16_to_f32(bb_raw), aa = bf16_to_f32(aa_raw);
    gb[tid][0] = -__expf(a_log) * softplus_g(aa + dtb);
    gb[tid][1] = round_bf16(1.f / (1.f + __expf(-bb)));
  }
  lds_only_barrier();
  // ---- 3. conv + SiLU (bf16 rounding at the conv output and at the SiLU output) ----
  for (int i = tid; i < T * GL_CH; i += 256) {
    const int r = i / GL_CH, lc = i % GL_CH;
    float acc = 0.f;
#pragma unroll
    for (int tau = 0; tau < GV_K; ++tau) acc = fmaf(bf16_to_f32(cw[lc][tau]), xin[r + tau][lc], acc);
    act[r][lc] = round_bf16(silu_g(round_bf16(acc)));
  }
  lds_only_barrier();
  // ---- 4. records of the new positions (k | v now, gamma, beta, 1/|k| in the scan) ----
  uint8_t* rep_out = a.rep + hout * a.S * GL_REC_BYTES;
  if (tid < T * 32)
    store_nt(rep_out + (size_t)(tid / 32) * GL_REC_BYTES + (tid % 32) * 16,
             gdn_record_kv(&act[tid / 32][GL_DK], tid % 32));
  // ---- 5. the committed state: the stored state + n replayed records, to the other half ----
  for (int j = 0; j < n; ++j)
    gdn_replay_one(S, reinterpret_cast<const uint8_t*>(rbuf) + (size_t)j * GL_REC_BYTES, row0, col0);
  {
    float* so = a.rec + hout * SS;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      store_nt(so + (size_t)(row0 + r) * GL_DK + col0,
               make_uint4(__float_as_uint(S[r][0]), __float_as_uint(S[r][1]),
                          __float_as_uint(S[r][2]), __float_as_uint(S[r][3])));
  }
  // ---- 6. the scan ----
  const float qscale = rsqrtf((float)GL_DK);
  for (int t = 0; t < T; ++t) {
    float kr[16], qr[16];
#pragma unroll
    for (int r = 0; r < 16; r += 4) {
      const float4 q4 = *reinterpret_cast<const float4*>(&act[t][row0 + r]);
      const float4 k4 = *reinterpret_cast<const float4*>(&act[t][GL_DK + row0 + r]);
      qr[r] = q4.x; qr[r + 1] = q4.y; qr[r + 2] = q4.z; qr[r + 3] = q4.w;
      kr[r] = k4.x; kr[r + 1] = k4.y; kr[r + 2] = k4.z; kr[r + 3] = k4.w;
    }
    float pa[4] = {0.f, 0.f, 0.f, 0.f}, pb[4] = {0.f, 0.f, 0.f, 0.f};
    float pkq = 0.f, pkk = 0.f, pqq = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pa[c] = fmaf(S[r][c], kr[r], pa[c]);
        pb[c] = fmaf(S[r][c], qr[r], pb[c]);
      }
      pkq = fmaf(kr[r], qr[r], pkq);
      pkk = fmaf(kr[r], kr[r], pkk);
      pqq = fmaf(qr[r], qr[r], pqq);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pa[c] = sum_lanes8(pa[c]);
      pb[c] = sum_lanes8(pb[c]);
    }
    pkq = sum_lanes8(pkq);
    pkk = sum_lanes8(pkk);
    pqq = sum_lanes8(pqq);
    const float rk = rsqrtf(pkk + 1e-6f);
    const float rq = rsqrtf(pqq + 1e-6f) * qscale;
    const float kq = pkq * rk * rq;
    const float gam = __expf(gb[t][0]), bet = gb[t][1];
    float vv[4], d[4], o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = act[t][2 * GL_DK + col0 + c];
    gdn_delta(d, pa, vv, gam, rk, bet);
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = gam * pb[c] * rq + d[c] * kq;
    if (rg == 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) obuf[t][col0 + c] = o[c];
    }
    if (tid == 0)
      store_nt(rep_out + (size_t)t * GL_REC_BYTES + 4 * GL_DK,
               make_uint4(__float_as_uint(gam), __float_as_uint(bet), __float_as_uint(rk), 0u));
    if (t + 1 < T) gdn_update(S, kr, rk, d, gam);   // the state after the last position is not kept
  }
  lds_only_barrier();
  // ---- 7. gated RMSNorm of each token's 128 outputs: 16 threads per token ----
  {
    const int i = tid >> 4, part = tid & 15;
    float ov[8], ss = 0.f;
    if (i < T) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ov[e] = round_bf16(obuf[i][part * 8 + e]);  // core output is a bf16 tensor
        ss += ov[e] * ov[e];
      }
    }
    ss = sum_lanes16(ss);
    if (i < T) {
      const float r = rsqrtf(ss / (float)GL_DK + a.eps);
      uint32_t od[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float y2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int ee = e + u;
          const float z = bf16_to_f32(zb[i][part * 8 + ee]);
          const float w = bf16_to_f32(nw[part * 8 + ee]);
          const float hn = round_bf16(ov[ee] * r);
          y2[u] = round_bf16(w * hn) * silu_g(z);
        }
        od[e >> 1] = f32_to_bf16(y2[0]) | ((uint32_t)f32_to_bf16(y2[1]) << 16);
      }
      *reinterpret_cast<uint4*>(a.out + ((size_t)b * T + i) * a.value_dim + (size_t)h * GL_DK +
                                part * 8) = make_uint4(od[0], od[1], od[2], od[3]);
    }
  }
}

// The committed state of each (sequence, head): the committed half's state with its first
// replay[b] records applied, in the register layout and arithmetic of the scans above.
// dst == nullptr: into the other half of rec (where a long call starts from); else into
// dst (B, Hv, Dk, Dv).
__global__ __launch_bounds__(256) void gdn_state_kernel(float* rec, const int32_t* rec_half,
                                                        const uint8_t* rep, const int32_t* replay,
                                                        int S, int Hv, float* dst) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = (lane >> 3) * 16, col0 = wave * 32 + (lane & 7) * 4;
  const int b = blockIdx.x / Hv, h = blockIdx.x % Hv;
  constexpr size_t SS = (size_t)GL_DK * GL_DK;
  const int half = rec_half[b] & 1;
  int n = replay[b];
  n = n < 0 ? 0 : (n > S ? S : n);
  const float* si = rec + ((size_t)(b * 2 + half) * Hv + h) * SS;
  float* so = dst ? dst + ((size_t)b * Hv + h) * SS : rec + ((size_t)(b * 2 + (half ^ 1)) * Hv + h) * SS;
  float St[16][4];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float4 f = *reinterpret_cast<const float4*>(si + (size_t)(row0 + r) * GL_DK + col0);
    St[r][0] = f.x; St[r][1] = f.y; St[r][2] = f.z; St[r][3] = f.w;
  }
  const uint8_t* rp = rep + ((size_t)(b * 2 + half) * Hv + h) * S * GL_REC_BYTES;
  for (int j = 0; j < n; ++j) gdn_replay_one(St, rp + (size_t)j * GL_REC_BYTES, row0, col0);
#pragma unroll
  for (int r = 0; r < 16; ++r)
    *reinterpret_cast<float4*>(so + (size_t)(row0 + r) * GL_DK + col0) =
        make_float4(St[r][0], St[r][1], St[r][2], St[r][3]);
}

}  // namespace lollm

using namespace lollm;

// Before a long call: the committed state into the other half (nothing to do on a fresh
// sequence, whose long call starts from zero).  Shared with lollm_gdn_layer_chunked.
int lollm::gdn_long_call_prologue(const GdnLayerArgs& a, int B, hipStream_t stream) {
  if (a.fresh) return LOLLM_OK;
  hipLaunchKernelGGL(gdn_state_kernel, dim3(B * a.Hv), dim3(256), 0, stream, a.rec, a.rec_half,
                     a.rep, a.replay, a.S, a.Hv, (float*)nullptr);
  return launch_status();
}

LOLLM_API int lollm_gdn_layer(const void* proj, long long proj_stride, const void* conv_w,
                              const float* A_log, const float* dt_bias, const void* norm_w,
                              void* win, const int32_t* conv_off, int win_rows, float* rec,
                              const int32_t* rec_half, void* rep, const int32_t* replay, int slots,
                              int fresh, void* out, int B, int T, int Hk, int Hv, int Dk, int Dv,
                              int conv_kernel, float eps, void* stream) {
  if (!proj || !conv_w || !A_log || !dt_bias || !norm_w || !win || !conv_off || !rec ||
      !rec_half || !rep || !replay || !out)
    return LOLLM_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return LOLLM_EINVAL;
  if (Dk != GL_DK || Dv != GL_DK || conv_kernel < 1 || conv_kernel > GL_KMAX) return LOLLM_EUNSUPPORTED;
  if (win_rows < conv_kernel - 1 || slots < 1) return LOLLM_EINVAL;
  const int key_dim = Hk * Dk, value_dim = Hv * Dv, C = 2 * key_dim + value_dim;
  if (proj_stride < (long long)C + value_dim + 2 * Hv || proj_stride % 8) return LOLLM_EINVAL;
  GdnLayerArgs a;
  a.proj = (const uint16_t*)proj; a.conv_w = (const uint16_t*)conv_w; a.A_log = A_log;
  a.dt_bias = dt_bias; a.norm_w = (const uint16_t*)norm_w; a.win = (uint16_t*)win;
  a.conv_off = conv_off; a.rec = rec; a.rec_half = rec_half; a.rep = (uint8_t*)rep;
  a.replay = replay; a.out = (uint16_t*)out;
  a.P = proj_stride; a.T = T; a.Hk = Hk; a.Hv = Hv; a.C = C; a.key_dim = key_dim;
  a.value_dim = value_dim; a.K = conv_kernel; a.W = win_rows; a.S = slots; a.fresh = fresh ? 1 : 0;
  a.eps = eps;
  const hipStream_t st = (hipStream_t)stream;
  const bool verify_form = T <= slots && slots <= GL_TC && conv_kernel == GV_K &&
                           conv_kernel - 1 + T <= win_rows && C % 8 == 0;
  if (verify_form) {
    hipLaunchKernelGGL(gdn_layer_verify_kernel, dim3(B * Hv), dim3(256), 0, st, a);
  } else if (T <= slots) {
    hipLaunchKernelGGL(gdn_layer_kernel<true>, dim3(B * Hv), dim3(256), 0, st, a);
  } else {
    const int rc = gdn_long_call_prologue(a, B, st);
    if (rc != LOLLM_OK) return rc;
    hipLaunchKernelGGL(gdn_layer_kernel<false>, dim3(B * Hv), dim3(256), 0, st, a);
  }
  return launch_status();
}

LOLLM_API int lollm_gdn_state(float* rec, const int32_t* rec_half, const void* rep,
                              const int32_t* replay, int slots, int B, int Hv, int Dk, int Dv,
                              float* out, void* stream) {
  if (!rec || !rec_half || !rep || !replay) return LOLLM_EINVAL;
  if (B <= 0 || Hv <= 0 || slots < 1) return LOLLM_EINVAL;
  if (Dk != GL_DK || Dv != GL_DK) return LOLLM_EUNSUPPORTED;
  hipLaunchKernelGGL(gdn_state_kernel, dim3(B * Hv), dim3(256), 0, (hipStream_t)stream, rec,
                     rec_half, (const uint8_t*)rep, replay, slots, Hv, out);
  return launch_status();
}

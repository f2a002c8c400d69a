// Fused elementwise / normalisation kernels of the qwen3_5 decoder step (gfx950).
//
//   rmsnorm      (src/qwen3_5/blocks.py:23-35) y = x * rsqrt(mean x^2 + eps) * (1 + w)
//                in fp32, optionally fused with the residual add of
//                modeling_qwen3_5.py:59-60 (x <- x + h, then y = norm(x))
//   mtp_input    (src/qwen3_5/mtp.py:61-73) the MTP head's fc input from token ids:
//                embedding lookup, both pre-fc RMSNorms and the concatenation
//   verify_input (src/qwen3_5/mtp.py:141-142 + modeling_qwen3_5.py embedding and layer
//                0's input norm) the verify block's ids, embedding rows and their norm
//   swiglu       (blocks.py:341-342) silu(gate) * up on a fused [gate | up] GEMM output
//   attn_prologue (blocks.py:214-227 + RoPE blocks.py:166-183 + kv.py:26-33):
//                split q_proj's per-head [query | gate], QK-norm (1 + w), partial
//                rotate-half RoPE at absolute positions len_b + t, and write k, v
//                post-RoPE / pre-GQA into the per-sequence KV cache
// Activations are bf16; intermediate arithmetic is fp32 with bf16 rounding at the
// points where the reference's bf16 tensors are materialised.
#include "common.h"

namespace lollm {

// One row of RMSNorm (RMS_THREADS threads; H % 8 == 0, vector loads of 8 bf16): x_row,
// optionally + h_row first (then written to xout_row when given), normalised into
// y_row.  Shared by every kernel that normalises a row so their bits agree.
__device__ __forceinline__ void rms_row(const uint16_t* __restrict__ x_row,
                                        const uint16_t* __restrict__ h_row,
                                        uint16_t* __restrict__ xout_row,
                                        const uint16_t* __restrict__ w,
                                        uint16_t* __restrict__ y_row, int H, float eps, float* red) {
  const uint4* x4 = reinterpret_cast<const uint4*>(x_row);
  const uint4* h4 = h_row ? reinterpret_cast<const uint4*>(h_row) : nullptr;
  const int n8 = H / 8;
  constexpr int MAXV = RMS_CHUNKS;  // H <= 8192
  // the norm weights are loaded with the row, not after the reduction: one memory round
  // trip per launch instead of two
  const uint4* w4 = reinterpret_cast<const uint4*>(w);
  uint4 wv[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * RMS_THREADS;
    wv[i] = c < n8 ? w4[c] : make_uint4(0, 0, 0, 0);
  }
  float v[MAXV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * RMS_THREADS;
    if (c < n8) {
      uint4 u = x4[c];
      uint32_t wd[4] = {u.x, u.y, u.z, u.w};
      uint32_t hd[4] = {0, 0, 0, 0};
      if (h4) { uint4 hv = h4[c]; hd[0] = hv.x; hd[1] = hv.y; hd[2] = hv.z; hd[3] = hv.w; }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float f = __uint_as_float((e & 1 ? wd[e >> 1] & 0xffff0000u : wd[e >> 1] << 16));
        if (h4) f = round_bf16(f + __uint_as_float((e & 1 ? hd[e >> 1] & 0xffff0000u : hd[e >> 1] << 16)));
        v[i][e] = f;
        ss += f * f;
      }
      if (h4 && xout_row) {
        uint4 o;
        o.x = f32_to_bf16(v[i][0]) | ((uint32_t)f32_to_bf16(v[i][1]) << 16);
        o.y = f32_to_bf16(v[i][2]) | ((uint32_t)f32_to_bf16(v[i][3]) << 16);
        o.z = f32_to_bf16(v[i][4]) | ((uint32_t)f32_to_bf16(v[i][5]) << 16);
        o.w = f32_to_bf16(v[i][6]) | ((uint32_t)f32_to_bf16(v[i][7]) << 16);
        reinterpret_cast<uint4*>(xout_row)[c] = o;
      }
    }
  }
  const float r = rms_rstd(ss, red, H, eps);
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * RMS_THREADS;
    if (c < n8) {
      const uint4 wu = wv[i];
      uint32_t wd[4] = {wu.x, wu.y, wu.z, wu.w};
      uint32_t od[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) od[e >> 1] = rms_out2(v[i][e], v[i][e + 1], r, wd[e >> 1]);
      reinterpret_cast<uint4*>(y_row)[c] = make_uint4(od[0], od[1], od[2], od[3]);
    }
  }
}

__global__ __launch_bounds__(RMS_THREADS) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                              const uint16_t* __restrict__ h,
                                                              uint16_t* __restrict__ x_out,
                                                              const uint16_t* __restrict__ w,
                                                              uint16_t* __restrict__ y, int H,
                                                              float eps) {
  __shared__ float red[RMS_THREADS / 64];
  const size_t row = blockIdx.x;
  rms_row(x + row * H, h ? h + row * H : nullptr, x_out ? x_out + row * H : nullptr, w, y + row * H,
          H, eps, red);
}

// The MTP head's input (src/qwen3_5/mtp.py:61-73 with the embedding lookup of the draft
// chain): out[b] = [RMSNorm_{1+w_emb}(table[tok[b]]) | RMSNorm_{1+w_hid}(hidden[b])],
// workgroup (b, half); the same row arithmetic as lollm_rmsnorm, so the bits equal the
// embedding + two norms + concatenation it replaces.  Ids are clamped into the table.
__global__ __launch_bounds__(RMS_THREADS) void mtp_input_kernel(const int32_t* __restrict__ tok,
                                                                long long tok_stride,
                                                                const uint16_t* __restrict__ hidden,
                                                                long long ldh,
                                                                const uint16_t* __restrict__ table,
                                                                int V,
                                                                const uint16_t* __restrict__ w_emb,
                                                                const uint16_t* __restrict__ w_hid,
                                                                uint16_t* __restrict__ out, int H,
                                                                float eps) {
  __shared__ float red[RMS_THREADS / 64];
  const int b = blockIdx.x;
  uint16_t* y = out + (size_t)b * 2 * H;
  if (blockIdx.y == 0) {
    int id = tok[(size_t)b * tok_stride];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    rms_row(table + (size_t)id * H, nullptr, nullptr, w_emb, y, H, eps, red);
  } else {
    rms_row(hidden + (size_t)b * ldh, nullptr, nullptr, w_hid, y + H, H, eps, red);
  }
}

// The verify block's input: ids[b] = [first[b], drafts[b, 0 .. k)] (T = k + 1 tokens),
// x[b, t] = table[ids[b, t]] (the embedding rows that open the residual stream) and
// y[b, t] = RMSNorm_{1+w}(x[b, t]) (layer 0's input norm, the row arithmetic of
// lollm_rmsnorm, so the bits equal the concatenation + embedding + norm it replaces);
// kv_len[b] = lengths[b] + T.  Workgroup (b, t); ids are clamped into the table for the
// lookup and stored as given.
__global__ __launch_bounds__(RMS_THREADS) void verify_input_kernel(
    const int32_t* __restrict__ first, const int32_t* __restrict__ drafts, int k,
    const uint16_t* __restrict__ table, int V, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ x, uint16_t* __restrict__ y, int32_t* __restrict__ ids,
    const int32_t* __restrict__ lengths, int32_t* __restrict__ kv_len, int H, float eps) {
  __shared__ float red[RMS_THREADS / 64];
  const int b = blockIdx.x, t = blockIdx.y, T = k + 1;
  const int id0 = t == 0 ? first[b] : drafts[(size_t)b * k + t - 1];
  const size_t row = (size_t)b * T + t;
  if (threadIdx.x == 0) {
    ids[row] = id0;
    if (t == 0 && kv_len) kv_len[b] = lengths[b] + T;
  }
  const int id = id0 < 0 ? 0 : (id0 >= V ? V - 1 : id0);
  const uint16_t* src = table + (size_t)id * H;
  for (int c = threadIdx.x; c < H / 8; c += RMS_THREADS)
    reinterpret_cast<uint4*>(x + row * H)[c] = reinterpret_cast<const uint4*>(src)[c];
  rms_row(src, nullptr, nullptr, w, y + row * H, H, eps, red);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }

// out[r, j] = bf16(bf16(silu(g)) * u) with g = gu[r, j], u = gu[r, F + j]
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ gu,
                                                     uint16_t* __restrict__ out, int F,
                                                     long long n8) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n8; i += (long long)gridDim.x * 256) {
    const long long r = i / (F / 8), c = i % (F / 8);
    const uint4 g = reinterpret_cast<const uint4*>(gu + r * 2 * F)[c];
    const uint4 u = reinterpret_cast<const uint4*>(gu + r * 2 * F + F)[c];
    const uint32_t gd[4] = {g.x, g.y, g.z, g.w}, ud[4] = {u.x, u.y, u.z, u.w};
    uint32_t od[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float g0 = __uint_as_float(gd[k] << 16), g1 = __uint_as_float(gd[k] & 0xffff0000u);
      const float u0 = __uint_as_float(ud[k] << 16), u1 = __uint_as_float(ud[k] & 0xffff0000u);
      od[k] = f32_to_bf16(round_bf16(silu_f(g0)) * u0) |
              ((uint32_t)f32_to_bf16(round_bf16(silu_f(g1)) * u1) << 16);
    }
    reinterpret_cast<uint4*>(out + r * F)[c] = make_uint4(od[0], od[1], od[2], od[3]);
  }
}

// One 256-thread workgroup per (token, head slot): slots [0, Hq) are query heads,
// [Hq, Hq + Hkv) key heads, [Hq + Hkv, Hq + 2 Hkv) value heads.  D == 256: one
// element per thread.
// QK-norm (1 + w) of one 256-value head vector (thread d holds x) followed by the partial
// rotate-half RoPE at position rpos (blocks.py:166-183,221-227), freq = inv_freq[d % (rd / 2)]
// for d < rd; returns thread d's output, a bf16 value.  The short-cache attention repeats
// this arithmetic so both give the same bits.  (red and xs are reused by the next call
// only after the barriers inside block_sum_f.)
__device__ __forceinline__ float qk_norm_rope(float x, float wv, float freq, int rpos, int rd,
                                              float eps, float* red, float* xs) {
  constexpr int D = 256;
  const int d = threadIdx.x;
  const float r = rsqrtf(block_sum_f<256>(x * x, red) / (float)D + eps);
  const float xn = round_bf16(x * r * (1.f + wv));  // QK-norm output (bf16 tensor)
  xs[d] = xn;
  __syncthreads();
  float y = xn;
  if (d < rd) {
    const int half = rd / 2;
    const float ang = (float)rpos * freq;
    const float c = round_bf16(cosf(ang)), s = round_bf16(sinf(ang));
    const float rot = d < half ? -xs[d + half] : xs[d - half];
    y = round_bf16(round_bf16(xn * c) + round_bf16(rot * s));
  }
  return y;
}

__global__ __launch_bounds__(256) void attn_prologue_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ inv_freq,
    const int32_t* __restrict__ lengths, const int32_t* __restrict__ rope_pos, int per_token,
    int T, int Hq, int Hkv, int rd, float eps,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ gate_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int max_len) {
  constexpr int D = 256;
  __shared__ float red[4];
  __shared__ float xs[D];
  const int bt = blockIdx.x, slot = blockIdx.y, d = threadIdx.x;
  const int b = bt / T, t = bt % T;
  const long long row_w = (long long)Hq * 2 * D + 2LL * Hkv * D;
  const uint16_t* src = qkv + (long long)bt * row_w;
  const int pos = lengths[b] + t;                          // cache row
  // RoPE position: the token's own entry of a (B, T) table, else a start per sequence + t
  const int rpos = per_token ? rope_pos[bt] : (rope_pos ? rope_pos[b] : lengths[b]) + t;
  if (slot >= Hq + Hkv) {  // value head: plain copy into the cache
    const int kvh = slot - Hq - Hkv;
    if (pos >= 0 && pos < max_len)
      vc[(((long long)b * Hkv + kvh) * max_len + pos) * D + d] = src[(long long)Hq * 2 * D + Hkv * D + kvh * D + d];
    return;
  }
  const bool is_q = slot < Hq;
  const uint16_t* xin = is_q ? src + (long long)slot * 2 * D : src + (long long)Hq * 2 * D + (slot - Hq) * D;
  if (is_q) gate_out[((long long)bt * Hq + slot) * D + d] = src[(long long)slot * 2 * D + D + d];
  // inv_freq[d % (rd / 2)] is loaded with the row, not after the norm's reduction
  const float freq = d < rd ? inv_freq[d % (rd / 2)] : 0.f;
  const float y = qk_norm_rope(bf16_to_f32(xin[d]), bf16_to_f32((is_q ? qn_w : kn_w)[d]), freq,
                               rpos, rd, eps, red, xs);
  if (is_q) {
    q_out[((long long)bt * Hq + slot) * D + d] = f32_to_bf16(y);
  } else if (pos >= 0 && pos < max_len) {
    const int kvh = slot - Hq;
    kc[(((long long)b * Hkv + kvh) * max_len + pos) * D + d] = f32_to_bf16(y);
  }
}

// Gated attention of one new token over a short cache (the MTP head's draft block:
// src/qwen3_5/mtp.py:61-73 with the chain's per-step cache) with the prologue fused:
// workgroup (sequence b, kv head) forms the new k (QK-norm + RoPE) and v, appends them at
// row lengths[b], forms its n_rep query heads and their gates exactly as the prologue
// does, then, one wave per query head, scores the first kv_len[b] rows (dot products in
// fp32, lane = 4 of the 256 dims), p = exp2(s c - max c) with c = scale log2(e),
// l = sum p, o = sum bf16(p) v / l, out = o sigmoid(gate) -- the arithmetic of the
// split-K kernel up to the order of the dot-product sums (blocks.py:208-235).
constexpr int AS_MAXL = 16;     // cache rows
constexpr int AS_MAXREP = 16;   // query heads per kv head

__device__ __forceinline__ float as_sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }

__global__ __launch_bounds__(256) void attn_small_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ inv_freq,
    const int32_t* __restrict__ lengths, const int32_t* __restrict__ rope_pos,
    const int32_t* __restrict__ kv_len, int Hq, int Hkv, int rd, float eps, float cl2,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int max_len, uint16_t* __restrict__ out) {
  constexpr int D = 256;
  __shared__ float redn[1 + AS_MAXREP][4];   // per-wave partial sums of the 1 + n_rep norms
  __shared__ float xsn[1 + AS_MAXREP][D];    // normed rows (k, then the query heads), for RoPE
  __shared__ float knew[D], vnew[D];
  __shared__ float qsh[AS_MAXREP][D], gsh[AS_MAXREP][D];
  const int b = blockIdx.x, kvh = blockIdx.y, d = threadIdx.x;
  const int lane = d & 63, wave = d >> 6;
  const int n_rep = Hq / Hkv;
  const long long row_w = (long long)Hq * 2 * D + 2LL * Hkv * D;
  const uint16_t* src = qkv + (long long)b * row_w;
  const int pos = lengths[b];
  const int rpos = rope_pos ? rope_pos[b] : pos;
  const size_t cbase = ((size_t)b * Hkv + kvh) * max_len;
  // every input of this (sequence, kv head) in one batch: k, v, the n_rep query heads and
  // their gates (the heads' norms below then run side by side, not one after another)
  const float kx = bf16_to_f32(src[(long long)Hq * 2 * D + kvh * D + d]);
  const uint16_t vb = src[(long long)Hq * 2 * D + Hkv * D + kvh * D + d];
  const float kw = bf16_to_f32(kn_w[d]), qw = bf16_to_f32(qn_w[d]);
  float qx[AS_MAXREP], gx[AS_MAXREP];
#pragma unroll
  for (int hr = 0; hr < AS_MAXREP; ++hr) {
    const int h = kvh * n_rep + (hr < n_rep ? hr : 0);
    qx[hr] = bf16_to_f32(src[(long long)h * 2 * D + d]);
    gx[hr] = bf16_to_f32(src[(long long)h * 2 * D + D + d]);
  }
  // the 1 + n_rep sums of squares, each with block_sum_f's order (the wave's xor tree, then
  // the four wave sums in order), so the k row has the prologue's bits
#pragma unroll
  for (int v = 0; v <= AS_MAXREP; ++v) {
    if (v > n_rep) break;
    const float x = v == 0 ? kx : qx[v - 1];
    float sq = x * x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
    if (lane == 0) redn[v][wave] = sq;
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v <= AS_MAXREP; ++v) {
    if (v > n_rep) break;
    const float t = 0.f + redn[v][0] + redn[v][1] + redn[v][2] + redn[v][3];
    const float r = rsqrtf(t / (float)D + eps);
    const float x = v == 0 ? kx : qx[v - 1];
    xsn[v][d] = round_bf16(x * r * (1.f + (v == 0 ? kw : qw)));  // QK-norm output (bf16 tensor)
  }
  __syncthreads();
  // partial rotate-half RoPE at rpos on the first rd dims (qk_norm_rope's arithmetic)
  float cs = 1.f, sn = 0.f;
  const int half = rd / 2;
  if (d < rd) {
    const float ang = (float)rpos * inv_freq[d % half];
    cs = round_bf16(cosf(ang));
    sn = round_bf16(sinf(ang));
  }
  auto rope = [&](int v) {
    const float xn = xsn[v][d];
    if (d >= rd) return xn;
    const float rot = d < half ? -xsn[v][d + half] : xsn[v][d - half];
    return round_bf16(round_bf16(xn * cs) + round_bf16(rot * sn));
  };
  {
    const uint16_t yb = f32_to_bf16(rope(0));
    knew[d] = bf16_to_f32(yb);
    vnew[d] = bf16_to_f32(vb);
    if (pos >= 0 && pos < max_len) {
      kc[(cbase + pos) * D + d] = yb;
      vc[(cbase + pos) * D + d] = vb;
    }
  }
#pragma unroll
  for (int hr = 0; hr < AS_MAXREP; ++hr) {
    if (hr >= n_rep) break;
    qsh[hr][d] = rope(1 + hr);
    gsh[hr][d] = gx[hr];
  }
  __syncthreads();
  int L = kv_len[b];
  L = L < 0 ? 0 : (L > max_len ? max_len : L);
  for (int hr = wave; hr < n_rep; hr += 4) {
    float q4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) q4[e] = qsh[hr][4 * lane + e];
    float sc[AS_MAXL];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < AS_MAXL; ++j) {
      sc[j] = -INFINITY;
      if (j < L) {
        float kv4[4];
        if (j == pos) {
#pragma unroll
          for (int e = 0; e < 4; ++e) kv4[e] = knew[4 * lane + e];
        } else {
          const uint2 u = *reinterpret_cast<const uint2*>(kc + (cbase + j) * D + 4 * lane);
          kv4[0] = __uint_as_float(u.x << 16); kv4[1] = __uint_as_float(u.x & 0xffff0000u);
          kv4[2] = __uint_as_float(u.y << 16); kv4[3] = __uint_as_float(u.y & 0xffff0000u);
        }
        float dot = q4[0] * kv4[0];
#pragma unroll
        for (int e = 1; e < 4; ++e) dot = fmaf(q4[e], kv4[e], dot);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) dot += __shfl_xor(dot, o, 64);
        sc[j] = dot;
        m = fmaxf(m, dot);
      }
    }
    const float base = m * cl2;
    float l = 0.f, o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < AS_MAXL; ++j) {
      if (j < L) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j], cl2, -base));
        l += p;
        const float pb = round_bf16(p);
        float vv4[4];
        if (j == pos) {
#pragma unroll
          for (int e = 0; e < 4; ++e) vv4[e] = vnew[4 * lane + e];
        } else {
          const uint2 u = *reinterpret_cast<const uint2*>(vc + (cbase + j) * D + 4 * lane);
          vv4[0] = __uint_as_float(u.x << 16); vv4[1] = __uint_as_float(u.x & 0xffff0000u);
          vv4[2] = __uint_as_float(u.y << 16); vv4[3] = __uint_as_float(u.y & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = fmaf(pb, vv4[e], o4[e]);
      }
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int h = kvh * n_rep + hr;
    uint32_t ow[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const float y0 = o4[e] * inv * as_sigmoid(gsh[hr][4 * lane + e]);
      const float y1 = o4[e + 1] * inv * as_sigmoid(gsh[hr][4 * lane + e + 1]);
      ow[e >> 1] = (uint32_t)f32_to_bf16(y0) | ((uint32_t)f32_to_bf16(y1) << 16);
    }
    *reinterpret_cast<uint2*>(out + ((size_t)b * Hq + h) * D + 4 * lane) = make_uint2(ow[0], ow[1]);
  }
}

// Greedy acceptance from the verify rows' argmax tokens (temperature 0): draft i of
// sequence b is kept while it equals the argmax of verify row i (the draft == true_next
// test of src/qwen3_5/mtp.py:141-155 with sample_next's argmax, src/generate.py:23-24), and
// the next pending token is the argmax of row a (the bonus row when all k are kept).
// One thread per sequence.
__global__ __launch_bounds__(64) void greedy_accept_kernel(const int32_t* __restrict__ amax,
                                                           const int32_t* __restrict__ drafts, int B,
                                                           int k, int32_t* __restrict__ n_acc,
                                                           int32_t* __restrict__ next_tok) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= B) return;
  const int32_t* am = amax + (size_t)b * (k + 1);
  int a = 0;
  while (a < k && drafts[(size_t)b * k + a] == am[a]) ++a;
  n_acc[b] = a;
  next_tok[b] = am[a];
}

// One workgroup per sequence: the bookkeeping that ends a speculative step.
__global__ __launch_bounds__(256) void spec_commit_kernel(
    const int32_t* __restrict__ verify_ids, const int32_t* __restrict__ n_acc,
    const int32_t* __restrict__ next_tok, int32_t* lengths, int32_t* rec_half, int32_t* replay,
    int32_t* conv_off,
    int32_t* pending, int32_t* out_tokens, int32_t* out_count, int cap,
    const uint16_t* __restrict__ hidden, uint16_t* __restrict__ h_last, int H, int T, int S,
    int W, long long* offset, int* hist, uint32_t* seen, int words) {
  const int b = blockIdx.x, tid = threadIdx.x;
  // every bookkeeping value is loaded before any store (the stores may alias the loads
  // as far as the compiler knows, which would otherwise order them one round trip each);
  // thread i < T holds verified position i
  const int len = lengths[b], rh = rec_half[b], co = conv_off[b], c = out_count[b];
  const int nt = next_tok[b];
  const int vid = tid < T ? verify_ids[b * T + tid] : 0;
  int a = n_acc[b];
  a = a < 0 ? 0 : (a > T - 1 ? T - 1 : a);
  const uint4* src = reinterpret_cast<const uint4*>(hidden + ((size_t)b * T + a) * H);
  uint4* dst = reinterpret_cast<uint4*>(h_last + (size_t)b * H);
  for (int i = tid; i < H / 8; i += 256) dst[i] = src[i];
  __syncthreads();   // every thread's loads of this sequence's counters precede the stores
  // keep a + 1 of the T positions
  if (tid <= a && c + tid < cap) out_tokens[(size_t)b * cap + c + tid] = vid;
  if (seen && tid >= 1 && tid <= a + 1) {
    // the repetition-penalty context: accepted drafts and the new pending token
    const int t = tid <= a ? vid : nt;
    if (t >= 0 && t < 32 * words) atomicOr(&seen[(size_t)b * words + (t >> 5)], 1u << (t & 31));
  }
  if (tid == 0) {
    lengths[b] = len + a + 1;
    rec_half[b] = (rh & 1) ^ 1;                     // the half the forward wrote,
    replay[b] = a + 1;                              // whose first a + 1 records are kept
    conv_off[b] = (co >= W ? 0 : W) + a + 1;
    out_count[b] = c + a + 1;
    pending[b] = nt;
    if (hist) atomicAdd(&hist[a], 1);
    if (b == 0) offset[0] += 1;
  }
}

}  // namespace lollm

using namespace lollm;

LOLLM_API int lollm_rmsnorm(const void* x, const void* residual, void* x_out, const void* w,
                            void* y, int rows, int H, float eps, void* stream) {
  if (!x || !w || !y || rows <= 0 || H <= 0) return LOLLM_EINVAL;
  if (H % 8 || H > 8192) return LOLLM_EUNSUPPORTED;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(RMS_THREADS), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)residual, (uint16_t*)x_out,
                     (const uint16_t*)w, (uint16_t*)y, H, eps);
  return launch_status();
}

LOLLM_API int lollm_mtp_input(const int32_t* tok, long long tok_stride, const void* hidden,
                              long long ld_hidden, const void* table, int vocab, const void* w_emb,
                              const void* w_hidden, void* out, int B, int H, float eps, void* stream) {
  if (!tok || !hidden || !table || !w_emb || !w_hidden || !out || B <= 0 || H <= 0 || vocab <= 0 ||
      tok_stride < 1)
    return LOLLM_EINVAL;
  if (H % 8 || H > 8192 || ld_hidden < H || ld_hidden % 8) return LOLLM_EUNSUPPORTED;
  hipLaunchKernelGGL(mtp_input_kernel, dim3(B, 2), dim3(RMS_THREADS), 0, (hipStream_t)stream, tok,
                     tok_stride, (const uint16_t*)hidden, ld_hidden, (const uint16_t*)table, vocab,
                     (const uint16_t*)w_emb, (const uint16_t*)w_hidden, (uint16_t*)out, H, eps);
  return launch_status();
}

LOLLM_API int lollm_verify_input(const int32_t* first, const int32_t* drafts, int k,
                                 const void* table, int vocab, const void* w, float eps,
                                 const int32_t* lengths, int32_t* ids, void* x, void* y,
                                 int32_t* kv_len, int B, int H, void* stream) {
  if (!first || !table || !w || !ids || !x || !y || B <= 0 || H <= 0 || vocab <= 0 || k < 0)
    return LOLLM_EINVAL;
  if ((k > 0 && !drafts) || (kv_len && !lengths)) return LOLLM_EINVAL;
  if (H % 8 || H > 8192 || B > 65535 || k + 1 > 65535) return LOLLM_EUNSUPPORTED;
  hipLaunchKernelGGL(verify_input_kernel, dim3(B, k + 1), dim3(RMS_THREADS), 0,
                     (hipStream_t)stream, first, drafts, k, (const uint16_t*)table, vocab,
                     (const uint16_t*)w, (uint16_t*)x, (uint16_t*)y, ids, lengths, kv_len, H, eps);
  return launch_status();
}

LOLLM_API int lollm_swiglu(const void* gate_up, void* out, int rows, int F, void* stream) {
  if (!gate_up || !out || rows <= 0 || F <= 0) return LOLLM_EINVAL;
  if (F % 8) return LOLLM_EUNSUPPORTED;
  const long long n8 = (long long)rows * (F / 8);
  const long long blocks = (n8 + 255) / 256;
  hipLaunchKernelGGL(swiglu_kernel, dim3(blocks < 4096 ? blocks : 4096), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)gate_up, (uint16_t*)out, F, n8);
  return launch_status();
}

LOLLM_API int lollm_attn_prologue(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                  const float* inv_freq, const int32_t* lengths,
                                  const int32_t* rope_pos, int rope_per_token, int B, int T,
                                  int Hq, int Hkv, int D, int rotary_dim, float eps, void* q_out,
                                  void* gate_out, void* k_cache, void* v_cache, int max_len,
                                  void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !lengths || !q_out || !gate_out || !k_cache || !v_cache)
    return LOLLM_EINVAL;
  if (rope_per_token && !rope_pos) return LOLLM_EINVAL;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || max_len <= 0) return LOLLM_EINVAL;
  if (D != 256 || rotary_dim < 0 || rotary_dim > D || rotary_dim % 2) return LOLLM_EUNSUPPORTED;
  if (rotary_dim > 0 && !inv_freq) return LOLLM_EINVAL;
  hipLaunchKernelGGL(attn_prologue_kernel, dim3(B * T, Hq + 2 * Hkv), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)qkv, (const uint16_t*)q_norm_w,
                     (const uint16_t*)k_norm_w, inv_freq, lengths, rope_pos, rope_per_token ? 1 : 0,
                     T, Hq, Hkv, rotary_dim, eps,
                     (uint16_t*)q_out, (uint16_t*)gate_out, (uint16_t*)k_cache,
                     (uint16_t*)v_cache, max_len);
  return launch_status();
}

LOLLM_API int lollm_attn_small(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                               const float* inv_freq, const int32_t* lengths,
                               const int32_t* rope_pos, const int32_t* kv_len, int B, int Hq,
                               int Hkv, int D, int rotary_dim, float eps, float scale,
                               void* k_cache, void* v_cache, int max_len, void* out,
                               void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !lengths || !kv_len || !k_cache || !v_cache || !out)
    return LOLLM_EINVAL;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || max_len <= 0) return LOLLM_EINVAL;
  if (D != 256 || rotary_dim < 0 || rotary_dim > D || rotary_dim % 2) return LOLLM_EUNSUPPORTED;
  if (max_len > AS_MAXL || Hq / Hkv > AS_MAXREP) return LOLLM_EUNSUPPORTED;
  if (rotary_dim > 0 && !inv_freq) return LOLLM_EINVAL;
  hipLaunchKernelGGL(attn_small_kernel, dim3(B, Hkv), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w,
                     inv_freq, lengths, rope_pos, kv_len, Hq, Hkv, rotary_dim, eps,
                     scale * 1.4426950408889634f, (uint16_t*)k_cache, (uint16_t*)v_cache, max_len,
                     (uint16_t*)out);
  return launch_status();
}

LOLLM_API int lollm_greedy_accept(const int32_t* argmax, const int32_t* drafts, int B, int k,
                                  int32_t* n_accepted, int32_t* next_token, void* stream) {
  if (!argmax || !n_accepted || !next_token || (k > 0 && !drafts)) return LOLLM_EINVAL;
  if (B <= 0 || k < 0) return LOLLM_EINVAL;
  hipLaunchKernelGGL(greedy_accept_kernel, dim3((B + 63) / 64), dim3(64), 0, (hipStream_t)stream,
                     argmax, drafts, B, k, n_accepted, next_token);
  return launch_status();
}

LOLLM_API int lollm_spec_commit(const int32_t* verify_ids, const int32_t* n_accepted,
                                const int32_t* next_token, int32_t* lengths, int32_t* rec_half,
                                int32_t* replay, int32_t* conv_off, int32_t* pending, int32_t* out_tokens,
                                int32_t* out_count, int out_cap, const void* hidden, void* h_last,
                                int B, int T, int H, int slots, int win_rows, long long* offset,
                                int32_t* accept_hist, uint32_t* seen, int seen_words,
                                void* stream) {
  if (!verify_ids || !n_accepted || !next_token || !lengths || !rec_half || !replay || !conv_off ||
      !pending || !out_tokens || !out_count || !hidden || !h_last || !offset)
    return LOLLM_EINVAL;
  if (B <= 0 || T <= 0 || H <= 0 || out_cap <= 0 || slots < T || win_rows <= 0) return LOLLM_EINVAL;
  if (T > 255) return LOLLM_EUNSUPPORTED;   // one thread per position and the pending token
  if (H % 8) return LOLLM_EUNSUPPORTED;
  if (seen && seen_words <= 0) return LOLLM_EINVAL;
  hipLaunchKernelGGL(spec_commit_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, verify_ids,
                     n_accepted, next_token, lengths, rec_half, replay, conv_off, pending, out_tokens,
                     out_count, out_cap, (const uint16_t*)hidden, (uint16_t*)h_last, H, T, slots,
                     win_rows, offset, accept_hist, seen, seen_words);
  return launch_status();
}

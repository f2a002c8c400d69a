/* Exact CPU restatement of the build's speculative-sampling rule -- TEST ORACLE ONLY.
 *
 * Never linked into the product.  The GPU sampler (lollm_amd/csrc/spec_sample.hip)
 * must reproduce every output of this file bit for bit on identical logits, drafts
 * and Philox keys.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off).
 *
 * What it restates:
 *   - generate.py:17-37 (`sample_next`): temperature, top-k (keep every token whose
 *     logit is >= the k-th largest), top-p (keep a token iff the probability mass of
 *     the tokens ranked strictly above it is <= top_p), greedy argmax at T <= 0
 *     (first index of the maximum, like torch.argmax).
 *   - The rejection rule required on top of mtp.py:144-155 (Leviathan et al. 2023,
 *     Chen et al. 2023): accept draft d at position i iff u * q_i(d) < p_i(d); at the
 *     first rejection draw from norm(max(0, p_i - q_i)); if all k drafts are accepted
 *     draw the bonus token from p_k.  With q one-hot (argmax drafts, mtp.py:138) this
 *     equals the reference's sample-and-match rule in distribution.
 *
 * Build-defined arithmetic (identical on CPU and GPU, no reduction-order freedom):
 *   - A logit's "sampling key" is its bf16 value with |x| <= 2^-16 flushed to 0.
 *     Tokens with equal keys are ties: top-k and top-p keep or drop them together.
 *   - Weight of a token: w = trunc(e * 2^39) with e = build_exp2((x - x_max) * c),
 *     c = inv_temperature * log2(e) in fp32; e is a Cody-Waite split 2^n * P(f) with
 *     a degree-7 Taylor polynomial of 2^f on f in [-1/2, 1/2] (Horner with fmaf).
 *     Tokens more than NBINS keys below the maximum key get weight 0.
 *   - Every sum of weights is an exact unsigned integer (u64 / u128), so the GPU may
 *     reduce in any order.  Top-p compares mass_above <= floor(W * P24 / 2^24) with
 *     P24 = trunc(top_p * 2^24).
 *   - Uniforms: Philox4x32-10 (Salmon et al., SC'11), key = (seed_lo, seed_hi),
 *     counter = (row, offset_lo, offset_hi, slot / 4), word = slot % 4, U = word >> 8
 *     (24-bit); u = U / 2^24.
 *   - Acceptance: U * wq(d) * Zp < 2^24 * wp(d) * Zq in 128-bit integers.
 *   - Draws: target = floor(U * Mass / 2^24); the token is the first (in id order)
 *     whose inclusive prefix mass exceeds target.  Residual weights are
 *     max(0, wp * Zq - wq * Zp), summed exactly in 128 bits.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

#define NBINS 8192
#define MAG0 0x3780 /* bf16 magnitude bits of 2^-16 */

/* ---------------------------------------------------------------- Philox4x32-10 */
static void philox_round(uint32_t c[4], const uint32_t k[2]) {
  uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
  uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
  uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k[0];
  uint32_t n1 = (uint32_t)p1;
  uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k[1];
  uint32_t n3 = (uint32_t)p0;
  c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
}

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
  uint32_t k[2] = {key[0], key[1]};
  for (int r = 0; r < 10; ++r) {
    if (r) { k[0] += 0x9E3779B9u; k[1] += 0xBB67AE85u; }
    philox_round(c, k);
  }
  memcpy(out, c, sizeof c);
}

uint32_t oracle_uniform_u24(uint64_t seed, uint64_t offset, uint32_t row, uint32_t slot) {
  uint32_t ctr[4] = {row, (uint32_t)offset, (uint32_t)(offset >> 32), slot >> 2};
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t o[4];
  oracle_philox4x32_10(ctr, key, o);
  return o[slot & 3] >> 8;
}

/* ------------------------------------------------------------- exp2 and weights */
float oracle_exp2(float t) { /* t in [-40, 0] */
  const float c1 = 0.693147180559945309f, c2 = 0.240226506959100712f,
              c3 = 0.0555041086648215800f, c4 = 0.00961812910762847717f,
              c5 = 0.00133335581464284434f, c6 = 1.54035303933816099e-4f,
              c7 = 1.52527338040598403e-5f;
  float n = rintf(t);
  float f = t - n;
  float p = c7;
  p = fmaf(p, f, c6);
  p = fmaf(p, f, c5);
  p = fmaf(p, f, c4);
  p = fmaf(p, f, c3);
  p = fmaf(p, f, c2);
  p = fmaf(p, f, c1);
  p = fmaf(p, f, 1.0f);
  return ldexpf(p, (int)n);
}

static inline int32_t skey(uint16_t b) {
  int32_t mag = b & 0x7FFF;
  int32_t mc = mag > MAG0 ? mag - MAG0 : 0;
  return (b & 0x8000) ? -mc : mc;
}

static inline float key_value(int32_t key) {
  if (key == 0) return 0.0f;
  uint32_t mag = (uint32_t)(key > 0 ? key : -key) + MAG0;
  uint32_t bits = (mag | (key < 0 ? 0x8000u : 0u)) << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint64_t oracle_weight(float x, float xmax, float c) {
  float t = (x - xmax) * c;
  if (!(t >= -40.0f)) return 0;
  float e = oracle_exp2(t);
  return (uint64_t)(e * 549755813888.0f); /* 2^39 */
}

/* ------------------------------------------------------------------- row stats */
typedef struct {
  int greedy;      /* 1: one-hot at argmax */
  int32_t argmax;  /* first index of the maximum bf16 value */
  int32_t kmax;    /* maximum sampling key */
  float xmax;      /* value of kmax */
  float c;         /* inv_temperature * log2(e) */
  int32_t cut;     /* keep iff kmax - key <= cut */
  uint64_t Z;      /* kept mass */
} RowStats;

static void row_stats(const uint16_t* x, int V, float inv_temp, int top_k, float top_p,
                      RowStats* s, uint32_t* counts /* NBINS scratch */) {
  int32_t am = 0;
  uint16_t best = 0;
  int32_t best_ord = -1;
  for (int i = 0; i < V; ++i) { /* raw order-preserving key for argmax */
    uint16_t b = x[i];
    int32_t ord = (b & 0x8000) ? (int32_t)(uint16_t)~b : (int32_t)(b | 0x8000);
    if (ord > best_ord) { best_ord = ord; am = i; best = b; }
  }
  (void)best;
  s->argmax = am;
  s->greedy = !(inv_temp > 0.0f);
  if (s->greedy) { s->Z = 1; s->cut = 0; return; }
  int32_t km = INT32_MIN;
  for (int i = 0; i < V; ++i) { int32_t k = skey(x[i]); if (k > km) km = k; }
  s->kmax = km;
  s->xmax = key_value(km);
  s->c = inv_temp * 1.44269504088896341f;
  memset(counts, 0, NBINS * sizeof(uint32_t));
  for (int i = 0; i < V; ++i) {
    int32_t d = km - skey(x[i]);
    if (d < NBINS) counts[d]++;
  }
  int32_t cut_k = NBINS - 1;
  if (top_k > 0) {
    uint64_t cum = 0;
    for (int d = 0; d < NBINS; ++d) {
      cum += counts[d];
      if (cum >= (uint64_t)top_k) { cut_k = d; break; }
    }
  }
  uint64_t W = 0;
  for (int d = 0; d <= cut_k; ++d)
    if (counts[d]) W += (uint64_t)counts[d] * oracle_weight(key_value(km - d), s->xmax, s->c);
  int32_t cut = cut_k;
  uint64_t Z = W;
  if (top_p > 0.0f && top_p < 1.0f) {
    uint32_t p24 = (uint32_t)(top_p * 16777216.0f);
    uint64_t tm = (uint64_t)(((u128)W * p24) >> 24);
    uint64_t cum = 0;
    for (int d = 0; d <= cut_k; ++d) {
      if (!counts[d]) continue;
      cum += (uint64_t)counts[d] * oracle_weight(key_value(km - d), s->xmax, s->c);
      if (cum > tm) { cut = d; Z = cum; break; }
    }
  }
  s->cut = cut;
  s->Z = Z;
}

static inline uint64_t token_weight(const RowStats* s, uint16_t b, int32_t tok) {
  if (s->greedy) return tok == s->argmax ? 1u : 0u;
  int32_t d = s->kmax - skey(b);
  if (d > s->cut) return 0;
  return oracle_weight(key_value(skey(b)), s->xmax, s->c);
}

/* inverse CDF over token ids: first token whose inclusive prefix weight > target */
static int32_t draw_row(const uint16_t* x, int V, const RowStats* s, uint32_t U) {
  if (s->greedy) return s->argmax;
  uint64_t target = (uint64_t)(((u128)U * s->Z) >> 24);
  uint64_t cum = 0;
  for (int i = 0; i < V; ++i) {
    cum += token_weight(s, x[i], i);
    if (cum > target) return i;
  }
  return V - 1; /* unreachable: target < Z */
}

/* floor(U * M / 2^24) exactly for M < 2^120 (U < 2^24). */
static inline u128 scaled_target(uint32_t U, u128 M) {
  return (u128)U * (M >> 24) + (((u128)U * (uint64_t)(M & 0xFFFFFFu)) >> 24);
}

/* residual weight max(0, wp * Zq - wq * Zp) of token t (exact, < 2^97) */
static inline u128 residual_weight(const RowStats* sp, const uint16_t* xp, const RowStats* sq,
                                   const uint16_t* xq, int32_t d, uint64_t Zq, int t) {
  uint64_t wpt = token_weight(sp, xp[t], t);
  uint64_t wqt = xq ? token_weight(sq, xq[t], t) : (uint64_t)(t == d);
  u128 l = (u128)wpt * Zq, r = (u128)wqt * sp->Z;
  return l > r ? l - r : 0;
}

/* ----------------------------------------------------------------- public API */
/* Row statistics exposed for tests: out = {argmax, kmax, cut, Z_lo, Z_hi}. */
int oracle_row_stats(const uint16_t* x, int V, float inv_temp, int top_k, float top_p,
                     int64_t* out) {
  uint32_t* counts = (uint32_t*)malloc(NBINS * sizeof(uint32_t));
  if (!counts) return -1;
  RowStats s;
  row_stats(x, V, inv_temp, top_k, top_p, &s, counts);
  free(counts);
  out[0] = s.argmax; out[1] = s.kmax; out[2] = s.cut;
  out[3] = (int64_t)s.Z;
  return 0;
}

/* Token weights of one row under its own filters (0 for dropped tokens). */
int oracle_row_weights(const uint16_t* x, int V, float inv_temp, int top_k, float top_p,
                       uint64_t* w) {
  uint32_t* counts = (uint32_t*)malloc(NBINS * sizeof(uint32_t));
  if (!counts) return -1;
  RowStats s;
  row_stats(x, V, inv_temp, top_k, top_p, &s, counts);
  free(counts);
  for (int i = 0; i < V; ++i) w[i] = token_weight(&s, x[i], i);
  return 0;
}

/* Draw one token per row; row r uses Philox row index (row_base + r) and `slot`. */
int oracle_sample_rows(const uint16_t* logits, int rows, int V, float inv_temp, int top_k,
                       float top_p, uint64_t seed, uint64_t offset, int row_base, int slot,
                       int32_t* out) {
  uint32_t* counts = (uint32_t*)malloc(NBINS * sizeof(uint32_t));
  if (!counts) return -1;
  for (int r = 0; r < rows; ++r) {
    RowStats s;
    const uint16_t* x = logits + (size_t)r * V;
    row_stats(x, V, inv_temp, top_k, top_p, &s, counts);
    uint32_t U = oracle_uniform_u24(seed, offset, (uint32_t)(row_base + r), (uint32_t)slot);
    out[r] = draw_row(x, V, &s, U);
  }
  free(counts);
  return 0;
}

/* Speculative acceptance for B sequences with k drafts each.
 * target: (B, k+1, V) bf16 bits; draft: (B, k, V) bf16 bits or NULL (one-hot q at
 * the draft token, i.e. argmax drafts); drafts: (B, k).  Outputs: n_accepted (B) in
 * 0..k and next_token (B): the residual draw at the first rejection, or the bonus
 * draw from target row k when all drafts are accepted. */
int oracle_spec_accept(const uint16_t* target, const uint16_t* draft, const int32_t* drafts,
                       int B, int k, int V, float inv_temp, int top_k, float top_p,
                       uint64_t seed, uint64_t offset, int32_t* n_accepted,
                       int32_t* next_token) {
  uint32_t* counts = (uint32_t*)malloc(NBINS * sizeof(uint32_t));
  if (!counts) return -1;
  for (int b = 0; b < B; ++b) {
    int a = 0;
    RowStats sp, sq;
    const uint16_t *xp = NULL, *xq = NULL;
    int rejected = 0;
    for (int i = 0; i < k; ++i) {
      int32_t d = drafts[b * k + i];
      xp = target + ((size_t)b * (k + 1) + i) * V;
      row_stats(xp, V, inv_temp, top_k, top_p, &sp, counts);
      uint64_t wp = token_weight(&sp, xp[d], d), Zp = sp.Z, wq, Zq;
      if (draft) {
        xq = draft + ((size_t)b * k + i) * V;
        row_stats(xq, V, inv_temp, top_k, top_p, &sq, counts);
        wq = token_weight(&sq, xq[d], d);
        Zq = sq.Z;
      } else {
        xq = NULL;
        wq = 1; Zq = 1;
      }
      uint32_t U = oracle_uniform_u24(seed, offset, (uint32_t)b, (uint32_t)i);
      u128 lhs = (u128)U * wq * Zp;
      u128 rhs = ((u128)wp * Zq) << 24;
      if (!(lhs < rhs)) { rejected = 1; break; }
      ++a;
    }
    uint32_t U = oracle_uniform_u24(seed, offset, (uint32_t)b, (uint32_t)k);
    int32_t tok;
    if (!rejected) {
      const uint16_t* xb = target + ((size_t)b * (k + 1) + k) * V;
      row_stats(xb, V, inv_temp, top_k, top_p, &sp, counts);
      tok = draw_row(xb, V, &sp, U);
    } else {
      int32_t d = drafts[b * k + a];
      uint64_t Zq = xq ? sq.Z : 1u;
      u128 R = 0;
      for (int t = 0; t < V; ++t)
        R += residual_weight(&sp, xp, &sq, xq, d, Zq, t);
      if (R == 0) {
        tok = draw_row(xp, V, &sp, U);
      } else {
        u128 target_mass = scaled_target(U, R);
        u128 cum = 0;
        tok = V - 1;
        for (int t = 0; t < V; ++t) {
          cum += residual_weight(&sp, xp, &sq, xq, d, Zq, t);
          if (cum > target_mass) { tok = t; break; }
        }
      }
    }
    n_accepted[b] = a;
    next_token[b] = tok;
  }
  free(counts);
  return 0;
}

/* ------------------------------------------------------------ repetition penalty */
/* generate.py:18-22 on one bf16 row: every distinct id of ids[0..n) in [0, V) becomes
 * bf16(x / penalty) if x > 0 else bf16(x * penalty), each computed in fp32 and rounded
 * to bf16 once, to nearest even -- what torch does for `s / p` and `s * p` on a bf16
 * tensor with a Python float (the fp32 opmath of its CPU kernels). */
static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

int oracle_repetition_penalty(uint16_t* row, int V, const int32_t* ids, int n, float penalty) {
  unsigned char* mark = (unsigned char*)calloc((size_t)V, 1);
  if (!mark) return 1;
  for (int i = 0; i < n; ++i)
    if (ids[i] >= 0 && ids[i] < V) mark[ids[i]] = 1;
  for (int v = 0; v < V; ++v) {
    if (!mark[v]) continue;
    uint32_t bits = (uint32_t)row[v] << 16;
    float x;
    memcpy(&x, &bits, 4);
    float y = x > 0.0f ? x / penalty : x * penalty;
    row[v] = f32_to_bf16_rne(y);
  }
  free(mark);
  return 0;
}

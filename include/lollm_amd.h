/* lollm_amd -- C ABI of the MI355X (gfx950) kernels for the qwen3_5 MTP
 * speculative-decode step.
 *
 * Conventions (every entry point):
 *   - Plain device pointers and sizes; no C++ or torch types cross the boundary.
 *   - Tensors are dense row-major in the shapes given; activations are bf16
 *     (dtype LOLLM_BF16, passed as uint16 bit patterns) or fp32 (LOLLM_F32).
 *   - `stream` is a hipStream_t (NULL = the default stream).  Launches are
 *     asynchronous; nothing allocates or frees device memory: the caller passes
 *     every output, snapshot and workspace buffer.
 *   - Return 0 on success, LOLLM_EINVAL for a bad argument, LOLLM_EUNSUPPORTED for
 *     a shape/dtype the kernels do not implement, LOLLM_EHIP_BASE + hipError_t for
 *     a launch failure.  lollm_strerror() names a code.
 */
#ifndef LOLLM_AMD_H
#define LOLLM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { LOLLM_BF16 = 0, LOLLM_F32 = 1 };
enum { LOLLM_OK = 0, LOLLM_EINVAL = 1, LOLLM_EUNSUPPORTED = 2, LOLLM_EHIP_BASE = 1000 };

const char* lollm_strerror(int code);
int lollm_abi_version(void);

/* Gated DeltaNet verify scan over T = 1 + k positions (the recurrent delta rule).
 *
 * Replaces: torch_recurrent_gated_delta_rule (src/qwen3_5/blocks.py:116-144) and,
 * for the T > 1 verify call, torch_chunk_gated_delta_rule (blocks.py:59-113, chosen
 * by blocks.py:316-322); snapshots replace the deep-copy rollback of kv.py:49-54 /
 * mtp.py:141,158.
 *
 *   q, k      (B, T, Hk, Dk)  dtype      v-head h reads qk-head h / (Hv / Hk)
 *   v         (B, T, Hv, Dv)  dtype
 *   g         (B, T, Hv)      fp32       log-decay; the state is scaled by exp(g)
 *   beta      (B, T, Hv)      dtype
 *   state     initial states (fp32, Dk x Dv each) or NULL for zeros: the state of
 *             (b, h) is state[((b * state_slots + slot_b) * Hv + h) * Dk * Dv] with
 *             slot_b = state_slot ? state_slot[b] : 0 (O(1) rollback: pass the
 *             previous call's snapshots with state_slot = accepted counts)
 *   out       (B, T, Hv, Dv)  dtype      o_t = S_t^T (q_t * q_scale)
 *   snapshots (B, T, Hv, Dk, Dv) fp32 or NULL: the state after each position
 *   final_state (B, Hv, Dk, Dv) fp32 or NULL: the state after position T-1 (may
 *             alias `state` when state_slots == 1 and state_slot == NULL)
 *   qk_l2norm  1: q and k are L2-normalised over Dk (eps 1e-6) inside the kernel
 * Supported: Dk == Dv == 128, Hv % Hk == 0, T >= 1. */
int lollm_gdn_verify(const void* q, const void* k, const void* v, const float* g,
                     const void* beta, const float* state, const int32_t* state_slot,
                     int state_slots, void* out, float* snapshots, float* final_state,
                     int B, int T, int Hk, int Hv, int Dk, int Dv, int dtype, int qk_l2norm,
                     float q_scale, void* stream);

/* Rollback materialisation: state_out[b, h] = snapshots[b, slot[b], h] for a
 * (B, T, Hv, Dk, Dv) fp32 snapshot buffer (O(1) callers skip this and index the
 * snapshots directly via lollm_gdn_verify's state_slot).
 * Replaces: the restore half of kv.py:49-54 + mtp.py:158. */
int lollm_gdn_select_state(const float* snapshots, const int32_t* slot, float* state_out,
                           int B, int T, int Hv, int Dk, int Dv, void* stream);

/* Gated GQA attention for T new queries per sequence over its KV cache.
 *
 * Replaces: attention() / torch_attention (src/attention.py:43-51,84-91), the KV
 * expansion _repeat_kv (src/qwen3_5/blocks.py:152-156,229) and the output gate
 * (blocks.py:235) of GatedAttention.forward; supersedes the Triton kv_fwd_kernel
 * (src/_triton_attn.py:37-111).
 *
 *   q        (B, T, Hq, D) bf16, after QK-norm and RoPE
 *   k_cache, v_cache  bf16; rows of D for (b, kv-head, position) at
 *            base + b * seq_stride + kvh * head_stride + pos * D   (elements)
 *   kv_len   (B) int32 keys per sequence INCLUDING the T new ones, which sit at
 *            positions kv_len - T .. kv_len - 1; query i attends positions
 *            <= kv_len - T + i (offset-causal)
 *   gate     (B, T, Hq * D) bf16 or NULL; out = attn * sigmoid(gate)
 *   out      (B, T, Hq * D) bf16
 *   workspace  split-K partials, lollm_attn_workspace_bytes() bytes (required)
 *   grid     workgroups of the balanced split (0: one per CU of the current device,
 *            at most 1024): the 128-key blocks of all (sequence, KV head) pairs are
 *            dealt out to them in equal contiguous ranges
 *   scale    softmax scale (D^-0.5)
 * Supported: D == 256, Hq / Hkv <= 32, B <= 512. */
long long lollm_attn_workspace_bytes(int B, int T, int Hq, int Hkv, int D, int max_len,
                                     int grid);
int lollm_attn_verify(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* kv_len, const void* gate, void* out, void* workspace,
                      long long workspace_bytes, int B, int T, int Hq, int Hkv, int D,
                      int max_len, long long seq_stride, long long head_stride, int grid,
                      float scale, void* stream);

/* Speculative-sampling acceptance over the full vocabulary for B sequences with k
 * drafts each, and the residual / bonus draw.
 *
 * Replaces: the accept/reject step of generate_mtp (src/qwen3_5/mtp.py:144-162) --
 * there sample-and-match with k = 1 -- by the rejection rule (accept draft d at
 * position i iff u q_i(d) < p_i(d); at the first rejection draw from
 * norm(max(0, p_i - q_i)); if all k are accepted draw the bonus from p_k), with p and
 * q formed as sample_next does (src/generate.py:17-37: temperature, top-k >= k-th
 * value, top-p on the mass ranked strictly above a token, greedy at T <= 0).
 *
 *   target   (B, k+1, V) bf16 logits of the verify pass
 *   draft    (B, k, V) bf16 draft logits, or NULL: q is one-hot at the draft token
 *            (argmax drafts, mtp.py:138)
 *   drafts   (B, k) int32 draft tokens
 *   inv_temperature  1/T as fp32 (0 = greedy); top_k (0 = off); top_p (>= 1 = off)
 *   seed, offset     Philox4x32-10 key and step counter; offset_dev, if not NULL, is a
 *            device pointer the offset is read from instead (for captured graphs)
 *   n_accepted (B) int32 in 0..k; next_token (B) int32
 *   workspace  lollm_spec_workspace_bytes(B, k, draft != NULL) bytes
 * Outputs are bit-exact to the integer specification in oracle/sampler_ref.c.
 * Supported: V % 8 == 0, T <= 1000, k <= 64. */
long long lollm_spec_workspace_bytes(int B, int k, int with_draft);
int lollm_spec_accept(const void* target, const void* draft, const int32_t* drafts, int B, int k,
                      int V, float inv_temperature, int top_k, float top_p, uint64_t seed,
                      uint64_t offset, const uint64_t* offset_dev, int32_t* n_accepted,
                      int32_t* next_token, void* workspace, long long workspace_bytes,
                      void* stream);

/* lollm_spec_accept with the target rows' maxima given: target_rowmax (B (k+1), rowmax_ld)
 * u16, row r's maximum order key of the bf16 logits being the largest of its first
 * rowmax_slots entries -- as lollm_gemm_logits writes them for the verify lm_head.  Each
 * target row is then read once (counts straight from the stream, no maximum pass);
 * results are bit-identical to lollm_spec_accept on the same logits.
 *
 * Replaces, with lollm_gemm_logits: the verify pass's logits, the repetition penalty and
 * the maximum / softmax / sort of sample_next (src/qwen3_5/mtp.py:141-155,
 * src/generate.py:17-37) as separate passes over the (B, 1 + k, V) logits. */
int lollm_spec_accept_rowmax(const void* target, const uint16_t* target_rowmax,
                             long long rowmax_ld, int rowmax_slots, const void* draft,
                             const int32_t* drafts, int B, int k, int V, float inv_temperature,
                             int top_k, float top_p, uint64_t seed, uint64_t offset,
                             const uint64_t* offset_dev, int32_t* n_accepted, int32_t* next_token,
                             void* workspace, long long workspace_bytes, void* stream);

/* lollm_spec_accept with no workspace argument and no device allocation, for callers that
 * cannot allocate: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  No counterpart in the reference.  The workspace is a fixed array inside the
 * library, LOLLM_SPEC_SCRATCH_BYTES on each device it runs on, held until the process
 * ends; a shape whose lollm_spec_workspace_bytes exceeds it returns LOLLM_EUNSUPPORTED
 * (1 MiB covers, e.g., B = 256 with k = 8 and sampled drafts).  Every call on one device
 * uses that device's array: calls that overlap in time on one device race.  Same
 * arguments, results and errors as lollm_spec_accept otherwise. */
#define LOLLM_SPEC_SCRATCH_BYTES (1 << 20)
int lollm_spec_accept_noalloc(const void* target, const void* draft, const int32_t* drafts, int B,
                              int k, int V, float inv_temperature, int top_k, float top_p,
                              uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                              int32_t* n_accepted, int32_t* next_token, void* stream);

/* One draw per row from its temperature / top-k / top-p distribution (the
 * multinomial of src/generate.py:37 on explicit uniforms); greedy rows return the
 * first argmax (generate.py:24).  Row r uses Philox row row_base + r and `slot`.
 * workspace: lollm_sample_workspace_bytes(rows) bytes. */
long long lollm_sample_workspace_bytes(int rows);
int lollm_sample_rows(const void* logits, int rows, int V, float inv_temperature, int top_k,
                      float top_p, uint64_t seed, uint64_t offset, const uint64_t* offset_dev,
                      int row_base, int slot, int32_t* out, void* workspace,
                      long long workspace_bytes, void* stream);

/* The 24-bit Philox uniforms the sampler uses: out[r * slots + s] = U(row r, slot s).
 * No reference counterpart (the reference draws implicitly with torch.multinomial). */
int lollm_philox_uniform_u24(uint64_t seed, uint64_t offset, int rows, int slots,
                             uint32_t* out, void* stream);

/* RMSNorm with (1 + w) scaling in fp32 (src/qwen3_5/blocks.py:23-35), fused with the
 * decoder's residual add (src/qwen3_5/modeling_qwen3_5.py:59-60) when residual !=
 * NULL: x_out = bf16(x + residual), y = norm(x_out).  x, residual, x_out, y: (rows,
 * H) bf16; w: (H) bf16.  Supported: H % 8 == 0, H <= 8192. */
int lollm_rmsnorm(const void* x, const void* residual, void* x_out, const void* w, void* y,
                  int rows, int H, float eps, void* stream);

/* The verify block's input in one kernel: the ids [pending, draft_1 .. draft_k] of the
 * verify pass (src/qwen3_5/mtp.py:141-142, `two`), their embedding rows
 * (modeling_qwen3_5.py:86) and layer 0's input RMSNorm (modeling_qwen3_5.py:48), with
 * lollm_rmsnorm's arithmetic, so the bits equal the concatenation + lookup + norm it
 * replaces.  first (B) int32, drafts (B, k) int32 (may be NULL when k == 0); ids (B, 1 + k)
 * int32 receives the ids as given (clamped into [0, vocab) only for the lookup); x, y
 * (B (1 + k), H) bf16 receive the embedding rows and their norm; kv_len (B) int32, if not
 * NULL, receives lengths[b] + 1 + k.  table (vocab, H) bf16, w (H) bf16.  Supported:
 * H % 8 == 0, H <= 8192. */
int lollm_verify_input(const int32_t* first, const int32_t* drafts, int k, const void* table,
                       int vocab, const void* w, float eps, const int32_t* lengths, int32_t* ids,
                       void* x, void* y, int32_t* kv_len, int B, int H, void* stream);

/* The MTP head's fc input from draft token ids (src/qwen3_5/mtp.py:61-73, with the
 * embedding lookup the draft chain does before it): out (B, 2H) bf16, row b =
 * [RMSNorm_{1+w_emb}(table[tok[b]]) | RMSNorm_{1+w_hidden}(hidden[b])], each half with
 * lollm_rmsnorm's arithmetic, so the bits equal the lookup + two norms + concatenation
 * it replaces.  tok[b * tok_stride] int32, clamped into [0, vocab); hidden (B, H) bf16 with row
 * stride ld_hidden; table (vocab, H) bf16.  Supported: H % 8 == 0, H <= 8192. */
int lollm_mtp_input(const int32_t* tok, long long tok_stride, const void* hidden, long long ld_hidden,
                    const void* table, int vocab, const void* w_emb, const void* w_hidden, void* out,
                    int B, int H, float eps, void* stream);

/* SwiGLU of blocks.py:341-342 on a fused [gate | up] projection: gate_up (rows, 2F)
 * bf16 -> out (rows, F) = bf16(bf16(silu(gate)) * up).  Supported: F % 8 == 0. */
int lollm_swiglu(const void* gate_up, void* out, int rows, int F, void* stream);

/* Attention prologue of GatedAttention.forward (blocks.py:214-227): from the fused
 * [q_proj | k_proj | v_proj] output qkv (B*T, Hq*2D + 2*Hkv*D) -- q_proj packing
 * [query | gate] per head -- write q (B, T, Hq, D) after QK-norm (1 + w) and partial
 * rotate-half RoPE (blocks.py:159-183) at positions rope_pos[b] + t (rope_pos NULL:
 * lengths[b] + t, the cache row; the MTP head defaults to positions 1..L, mtp.py:66-67) or,
 * with rope_per_token != 0, at rope_pos[b * T + t] (a (B, T) table: MTP.forward's explicit
 * positions vector, mtp.py:61-67), the gate (B, T, Hq*D), and k (normed, roped) / v into
 * the caches at (b, kvh, lengths[b] + t) (kv.py:26-33 without the concatenation).
 * inv_freq: (rotary_dim / 2) fp32.  Supported: D == 256. */
int lollm_attn_prologue(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                        const float* inv_freq, const int32_t* lengths, const int32_t* rope_pos,
                        int rope_per_token, int B, int T, int Hq,
                        int Hkv, int D, int rotary_dim, float eps, void* q_out, void* gate_out,
                        void* k_cache, void* v_cache, int max_len, void* stream);

/* Gated attention of one new token per sequence over a short cache, prologue fused
 * (GatedAttention.forward, blocks.py:208-235, for the MTP head's draft block with the
 * chain's per-step cache, mtp.py:61-73): from the fused qkv (B, Hq*2D + 2*Hkv*D) of the
 * token, the new k / v are formed and appended at row lengths[b] exactly as
 * lollm_attn_prologue does, then out (B, Hq*D) bf16 = softmax(q k^T scale) v *
 * sigmoid(gate) over the first kv_len[b] cache rows, with lollm_attn_verify's arithmetic
 * up to the order of the dot-product sums.  rope_pos as in lollm_attn_prologue.
 * Supported: D == 256, max_len <= 16, Hq / Hkv <= 16. */
int lollm_attn_small(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                     const float* inv_freq, const int32_t* lengths, const int32_t* rope_pos,
                     const int32_t* kv_len, int B, int Hq, int Hkv, int D, int rotary_dim, float eps,
                     float scale, void* k_cache, void* v_cache, int max_len, void* out, void* stream);

/* Few-row weight GEMM: y = x W^T for x with M <= 64 rows (the verify pass over
 * B x (1 + k) positions, the draft pass over B), bf16 in / fp32 accumulate / bf16 out.
 *
 * Replaces: the bias-free nn.Linear projections of the decoder and MTP head when the
 * rows are few -- in_proj_qkv|z|b|a and out_proj (src/qwen3_5/blocks.py:255-262,
 * 309-329), q|k|v_proj and o_proj (blocks.py:199-236), gate|up and down_proj
 * (blocks.py:332-342), lm_head (modeling_qwen3_5.py:73,99) and mtp.fc (mtp.py:61-73).
 *
 * lollm_gemm_tile_weights re-lays an (N, K) row-major bf16 weight once, at load, into
 * 1 KB blocks in MFMA operand order (N * K elements): block (t, s) for rows 16 t ..
 * 16 t + 15 and k 32 s .. 32 s + 31 at element (t * K / 32 + s) * 512, lane L = 16 g + r
 * holding row 16 t + r, k 32 s + 8 g .. + 8.  epilogue 1 (SwiGLU) takes W = [gate;
 * up] (N = 2F) and interleaves gate / up rows 8 by 8.
 *
 * lollm_gemm: A (M, lda) bf16; Wt the tiled weight; C (M, ldc) bf16 with N columns, or
 * N / 2 = bf16(bf16(silu(bf16(x gate^T))) * bf16(x up^T)) for epilogue 1
 * (blocks.py:341-342 with the reference's bf16 tensors); workspace: fp32 pieces of the
 * column groups cut between workgroups, merged by a second kernel of the same call,
 * lollm_gemm_workspace_bytes(M, N, K, grid) bytes (calls sharing one workspace must
 * not overlap in time); grid: workgroups (0 = two per CU, at most 1024).
 * Supported: 1 <= M <= 64, N % 64 == 0, K % 128 == 0, lda % 8 == 0. */
int lollm_gemm_tile_weights(const void* W, void* Wt, int N, int K, int epilogue, void* stream);
long long lollm_gemm_workspace_bytes(int M, int N, int K, int grid);
int lollm_gemm(const void* A, long long lda, const void* Wt, void* C, long long ldc, int M,
               int N, int K, int epilogue, void* workspace, long long workspace_bytes, int grid,
               void* stream);

/* The greedy draft pick fused into the lm_head GEMM (src/qwen3_5/mtp.py:138: the draft
 * is the argmax of the MTP head's logits; the reference computes the (B, V) logits with
 * model.lm_head and argmaxes them): out[r * out_stride] = argmax_n of row r of
 * A W^T, where each product is rounded to bf16 exactly as lollm_gemm writes it and ties
 * go to the lowest column -- the same token as lollm_gemm followed by the greedy
 * lollm_sample_rows, without materialising the logits.  Wt tiled with epilogue 0;
 * shapes as lollm_gemm; workspace from lollm_gemm_argmax_workspace_bytes. */
long long lollm_gemm_argmax_workspace_bytes(int M, int N, int K, int grid);
int lollm_gemm_argmax(const void* A, long long lda, const void* Wt, int M, int N, int K,
                      int32_t* out, long long out_stride, void* workspace, long long workspace_bytes,
                      int grid, void* stream);

/* The lm_head with the repetition penalty and the sampler's row maxima fused: C (M, ldc)
 * bf16 = A W^T (as lollm_gemm, 64-column groups), each logit of row m = (s, t) with
 * s = m / T penalised in place when its token is in seen[s] (seen_words u32 words per
 * row, bit tok % 32 of word tok / 32) or among extra[s * extra_stride + j] for
 * j < n_extra0 + t (seen NULL: no penalty) -- x > 0 ? x / penalty : x * penalty in fp32
 * on the bf16 logit, rounded once, the bits of lollm_repetition_penalty -- and rowmax
 * (M, rowmax_ld) u16 with, per row, lollm_gemm_rowmax_slots(grid) slots whose largest
 * entry is the maximum order key of the stored row (order key of bf16 bits b:
 * b & 0x8000 ? ~b & 0xFFFF : b | 0x8000).  Every slot is written by every call.
 *
 * Replaces: lm_head (src/qwen3_5/modeling_qwen3_5.py:99) on the verify rows, the
 * repetition penalty of sample_next (src/generate.py:18-22), and the maximum pass of its
 * softmax (generate.py:26-31), which lollm_spec_accept_rowmax then skips.
 * Workspace and supported shapes as lollm_gemm; with extra, n_extra0 + T - 1 <= 8. */
int lollm_gemm_rowmax_slots(int grid);
int lollm_gemm_logits(const void* A, long long lda, const void* Wt, int M, int N, int K, void* C,
                      long long ldc, uint16_t* rowmax, long long rowmax_ld, const uint32_t* seen,
                      int seen_words, const int32_t* extra, int extra_stride, int n_extra0, int T,
                      float penalty, void* workspace, long long workspace_bytes, int grid,
                      void* stream);

/* A projection that feeds the residual stream, with the residual add and the next
 * RMSNorm fused into the GEMM's second kernel: C = A W^T (as lollm_gemm, epilogue 0),
 * x_out = bf16(C + residual), y = RMSNorm_{1+w}(x_out) (lollm_rmsnorm's arithmetic).
 *
 * Replaces: o_proj (src/qwen3_5/blocks.py:236), out_proj (blocks.py:326) and down_proj
 * (blocks.py:342) followed by the residual adds and norms of the decoder layer
 * (modeling_qwen3_5.py:59-60) -- `x = x + h; y = post_attention_layernorm(x)` and
 * `x = x + mlp(...)` feeding the next layer's input_layernorm or the final norm.
 *
 * C (M, N) bf16 scratch; residual, x_out, y (M, N) bf16 contiguous (x_out may alias
 * residual; residual NULL: x_out = bf16(x W^T), no add -- the MTP fc followed by the MTP
 * layer's input_layernorm, src/qwen3_5/mtp.py:61-73); norm_w (N) bf16; workspace as
 * lollm_gemm.  Supported: N <= 8192 and at
 * least as many (64-column, 128-k) units as workgroups, else LOLLM_EUNSUPPORTED. */
int lollm_gemm_rmsnorm(const void* A, long long lda, const void* Wt, int M, int N, int K,
                       const void* residual, const void* norm_w, float eps, void* C, void* x_out,
                       void* y, void* workspace, long long workspace_bytes, int grid, void* stream);

/* The Gated DeltaNet mixer from the in_proj outputs to the gated-norm output
 * (GatedDeltaNet.forward, blocks.py:288-329, between in_proj and out_proj):
 * causal conv + SiLU, beta / g gating, L2-normalised delta-rule scan, gated RMSNorm.
 *   proj      (B, T, proj_stride) bf16: [qkv (conv_dim) | z (Hv*Dv) | b (Hv) | a (Hv)]
 *   conv_w    (conv_dim, conv_kernel) bf16; A_log, dt_bias (Hv) fp32; norm_w (Dv) bf16
 *   win       (B, 2 * win_rows, conv_dim) bf16, two window halves: the committed conv
 *             state is rows conv_off[b] .. conv_off[b] + conv_kernel - 2; the call
 *             writes the other half (base h = 0 or win_rows): if conv_kernel - 1 + T
 *             <= win_rows the whole window [state | raw x_0..x_{T-1}] at rows h.. (state
 *             after c committed tokens = rows h + c ..), else the final state at rows h..
 *   rec       (B, 2, Hv, Dk, Dv) fp32 and rep (B, 2, Hv, slots, 4 Dk + 16) bytes: two
 *             halves of recurrent state + replay records.  The committed state is half
 *             rec_half[b]'s state with its first replay[b] records applied (ignored when
 *             fresh: zero state).  The call writes only the other half: if T <= slots,
 *             the committed state and the records of its T positions (k and v after the
 *             conv as bf16, then fp32 exp(g), beta, 1/|k|), so the state after position t
 *             is that half with replay = t + 1; else (long call) the final state, with
 *             replay = 0.  The committed half is never written.
 *   out       (B, T, Hv*Dv) bf16
 * Replaces: GatedDeltaNet._conv, the gating, torch_chunk_gated_delta_rule /
 * torch_recurrent_gated_delta_rule and RMSNormGated (blocks.py:38-51,59-144,268-329),
 * and the speculative deep copy of the linear state (kv.py:49-54).
 * Supported: Dk == Dv == 128, conv_kernel <= 4. */
int lollm_gdn_layer(const void* proj, long long proj_stride, const void* conv_w,
                    const float* A_log, const float* dt_bias, const void* norm_w, void* win,
                    const int32_t* conv_off, int win_rows, float* rec, const int32_t* rec_half,
                    void* rep, const int32_t* replay, int slots, int fresh, void* out, int B, int T,
                    int Hk, int Hv, int Dk, int Dv, int conv_kernel, float eps, void* stream);

/* The committed recurrent state of every (sequence, head) of one GDN layer -- half
 * rec_half[b] of rec with its first replay[b] records of rep applied, as lollm_gdn_layer
 * lays them out -- into out (B, Hv, Dk, Dv) fp32; with out == NULL, into the other half
 * of rec instead (after which rec_half[b] ^= 1, replay[b] = 0 names the same state with
 * no records).  Replaces reading and replacing the recurrent state of the cache
 * (src/qwen3_5/kv.py:39-44). */
int lollm_gdn_state(float* rec, const int32_t* rec_half, const void* rep, const int32_t* replay,
                    int slots, int B, int Hv, int Dk, int Dv, float* out, void* stream);

/* The same layer for long calls (prefill) with the delta rule in its chunked parallel
 * form: torch_chunk_gated_delta_rule (src/qwen3_5/blocks.py:59-113), which the reference
 * runs for every T > 1 call (blocks.py:316-322), fused with the conv / gating / norm of
 * lollm_gdn_layer.  Chunks of 64 tokens on bf16 MFMA, each fp32 operand entering as a
 * hi + lo pair of bf16 values (relative error near 2^-17), the triangular solve's
 * off-diagonal blocks on fp32 MFMA; the L2 norm of q and k (blocks.py:124-127) is
 * applied as fp32 scales, as the recurrent kernels do.  Same
 * arguments and the same long-call placement as lollm_gdn_layer: the final state in
 * the half not holding rec_half[b], the final K-1 raw inputs in rows 0 .. K-2
 * of the window half not holding conv_off[b].  Supported: conv_kernel 4, T > slots,
 * K - 1 + T > win_rows (the call does not fit a window half), else LOLLM_EUNSUPPORTED. */
int lollm_gdn_layer_chunked(const void* proj, long long proj_stride, const void* conv_w,
                            const float* A_log, const float* dt_bias, const void* norm_w,
                            void* win, const int32_t* conv_off, int win_rows, float* rec,
                            const int32_t* rec_half, void* rep, const int32_t* replay, int slots,
                            int fresh, void* out, int B, int T, int Hk, int Hv, int Dk, int Dv,
                            int conv_kernel, float eps, void* stream);

/* Greedy acceptance (temperature 0) without the verify logits: argmax (B, k + 1) int32
 * holds the argmax token of each verify row (lollm_gemm_argmax on the lm_head, same
 * token as lollm_gemm + the greedy sampler); n_accepted[b] = the number of leading drafts
 * (B, k) equal to their row's argmax, next_token[b] = the argmax of row n_accepted[b].
 * Replaces the draft == true_next test and the next sample_next of src/qwen3_5/mtp.py
 * :141-155 at temperature 0 (sample_next's argmax, src/generate.py:23-24); with
 * lollm_gemm_argmax it keeps the (B, 1 + k, V) verify logits from being materialised. */
int lollm_greedy_accept(const int32_t* argmax, const int32_t* drafts, int B, int k,
                        int32_t* n_accepted, int32_t* next_token, void* stream);

/* End of one speculative step, per sequence b with a = n_accepted[b] (of T - 1
 * drafts): keep a + 1 of the T verified positions (lengths += a + 1, GDN state half =
 * the written half with replay = a + 1 records, conv window offset = written half + a
 * + 1, with the halves of lollm_gdn_layer: slots / win_rows) -- the O(1) form of the
 * snapshot/restore
 * of src/qwen3_5/mtp.py:141,156-162), append verify_ids[b, 0..a] to out_tokens (cap
 * columns) at out_count[b], copy hidden[b, a] (B, T, H) to h_last (B, H) (the MTP
 * input, mtp.py:155,162), set pending = next_token, increment *offset (the
 * sampler's Philox step counter) and, if accept_hist != NULL, accept_hist[a] (T
 * counters: the accepted-length histogram) and, if seen != NULL, mark the accepted drafts
 * verify_ids[b, 1..a] and the new pending token in the (B, seen_words) repetition-penalty
 * bitmaps (the context.append calls of mtp.py:129,150).  No reference counterpart as one
 * call: it folds the reference's per-step host bookkeeping into one kernel so a step needs
 * no sync.  The caller guarantees out_count[b] + T <= out_cap and lengths[b] + T <= the
 * cache length before each step (the Python host keeps upper bounds and raises first). */
int lollm_spec_commit(const int32_t* verify_ids, const int32_t* n_accepted,
                      const int32_t* next_token, int32_t* lengths, int32_t* rec_half,
                      int32_t* replay, int32_t* conv_off, int32_t* pending, int32_t* out_tokens, int32_t* out_count,
                      int out_cap, const void* hidden, void* h_last, int B, int T, int H,
                      int slots, int win_rows, long long* offset, int32_t* accept_hist,
                      uint32_t* seen, int seen_words, void* stream);

/* Repetition penalty of sample_next (src/generate.py:18-22), in place on bf16 logits, before
 * any sampler kernel reads them: every token of a row's penalty set becomes
 * bf16(x / penalty) if x > 0 else bf16(x * penalty), each computed in fp32 and rounded once
 * (torch's arithmetic on bf16 tensors), each token once however often it occurs
 * (the reference's set(prev_ids)).
 *   logits  B * T rows of V bf16, row (b, t) at logits + (b * T + t) * ld
 *   seen    (B, words) uint32, words >= ceil(V / 32): bit v of row b set iff token v is in
 *           sequence b's context (prompt, emitted tokens, the pending token)
 *   extra   (B, extra_stride) int32 or NULL: row (b, t) also penalises
 *           extra[b * extra_stride + 0 .. n_extra0 + t - 1] -- the drafts verified before
 *           position t, which the reference appends to its context (mtp.py:150) before it
 *           samples the next position -- skipping tokens already in the bitmap
 * Replaces: the index / where / scatter of generate.py:18-22 over set(prev_ids), on the
 * device and inside a captured step.  penalty > 0; B * T <= 65535. */
int lollm_repetition_penalty(void* logits, long long ld, int B, int T, int V, const uint32_t* seen,
                             int words, const int32_t* extra, int extra_stride, int n_extra0,
                             float penalty, void* stream);

/* seen[b] |= { tok[b * tok_stride + i] : i < n } for b < B (tokens outside [0, V) ignored):
 * builds the repetition-penalty context of lollm_repetition_penalty from a prompt or a
 * token list.  Replaces: the context list of src/generate.py:45,56 / mtp.py:108,129. */
int lollm_seen_mark(uint32_t* seen, int words, int B, const int32_t* tok, long long tok_stride,
                    int n, int V, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOLLM_AMD_H */

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

#ifdef __cplusplus
}
#endif

#endif /* LOLLM_AMD_H */

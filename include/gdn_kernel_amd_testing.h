/*
 * gdn_kernel_amd testing entry points (MI355X / gfx950).
 *
 * Not part of the drop-in surface and with no counterpart in the reference: these
 * exist for tests and tuning.  gdn_prefill_fault_injection drives the prefill
 * kernel's failure handling from the host: the prefill workgroup runs two roles
 * that hand chunks to each other through bounded waits; a wait that gives up
 * raises a workgroup abort flag after which every later wait returns at once, so
 * the kernel always finishes (with wrong results) instead of hanging.  The
 * *_with_variant decode entry points select a launch shape explicitly.
 */
#ifndef GDN_KERNEL_AMD_TESTING_H
#define GDN_KERNEL_AMD_TESTING_H

#include "gdn_kernel_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * gdn_prefill with three testing hooks (all arguments as gdn_prefill):
 *   spin_limit   polls before a hand-off wait gives up (0: the production default,
 *                about 70 ms); must be >= 0.
 *   ready_chunks > 0: the producer waves signal "chunk ready" only for the first
 *                ready_chunks chunks of each workgroup, so the consumer waves'
 *                wait for chunk ready_chunks + 1 can only end by giving up;
 *                0: no limit.  Must be >= 0.
 *   aborts       device uint32 counter (or NULL): incremented once by each
 *                wavefront whose wait gives up.  The caller clears it.
 * With spin_limit = ready_chunks = 0 and aborts = NULL this is gdn_prefill.
 */
int gdn_prefill_fault_injection(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                                const float* state, const float* A_log, const gdn_bf16* a,
                                const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                                int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                                double scale, gdn_bf16* output, float* new_state,
                                int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                                int32_t head_dim_k, int32_t head_dim_v, int32_t spin_limit,
                                int32_t ready_chunks, uint32_t* aborts, void* stream);

/*
 * Decode with an explicit launch shape instead of the batch-size heuristic, so that
 * tests can check every compiled shape and tuning runs can time them.  Arguments as
 * gdn_decode / gdn_decode_pooled plus `variant` in [0, gdn_decode_num_variants()):
 * a (rows per wavefront, wavefronts per workgroup, nontemporal state access) shape
 * of the decode kernel.  Out-of-range variants return GDN_ERR_INVALID_ARGUMENT.
 */
int gdn_decode_num_variants(void);

int gdn_decode_with_variant(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                            const float* state, const float* A_log, const gdn_bf16* a,
                            const float* dt_bias, const gdn_bf16* b, double scale,
                            gdn_bf16* output, float* new_state, int64_t batch,
                            int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                            int32_t head_dim_k, int32_t head_dim_v, int32_t variant,
                            void* stream);

int gdn_decode_pooled_with_variant(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                                   float* state_pool, int64_t pool_slots,
                                   const int32_t* state_indices, const float* A_log,
                                   const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                                   double scale, gdn_bf16* output, int64_t batch,
                                   int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                                   int32_t head_dim_k, int32_t head_dim_v, int32_t variant,
                                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_KERNEL_AMD_TESTING_H */

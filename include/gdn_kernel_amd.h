/*
 * gdn_kernel_amd -- C ABI of the MI355X (gfx950) Gated DeltaNet decode and
 * varlen chunked prefill kernels.
 *
 * Every entry point takes raw device pointers, explicit sizes and a HIP stream
 * passed as an opaque pointer (hipStream_t; NULL = the default stream).  All
 * tensors are dense row-major (C-contiguous) in the layouts documented per
 * function; bf16 tensors are raw 16-bit bf16 bit patterns.  Launches are
 * asynchronous on the given stream.
 *
 * Synchronisation, allocation and state (what each entry point does beyond its
 * outputs):
 *   - No entry point allocates device memory (no hipMalloc / hipFree, no library
 *     routine that allocates).
 *   - gdn_prefill_giveups and gdn_decode_pool_conflicts synchronise the current
 *     device (hipDeviceSynchronize) before they read their device counter; no other
 *     entry point synchronises the device, a stream or the host.
 *   - Static device memory: every device the library's code is loaded onto holds,
 *     from load until the process ends, gdn_static_device_bytes() bytes:
 *     GDN_PREFILL_DROPIN_SCRATCH_BYTES (gdn_prefill's scratch) +
 *     GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES (gdn_prefill_no_alloc's) + 12 bytes of
 *     device counters (192 MiB in all), whether or not a prefill ever runs.
 *     Torch's allocator does not see it.
 *   - Per-device host state: gdn_prefill and gdn_prefill_no_alloc each keep, per
 *     device and for their own scratch array, the array's address, a mutex and one
 *     event (created on first use and kept) that orders their two-kernel launches
 *     on that device (each such launch waits, on its stream, for the event the
 *     previous one recorded).  The two device counters (prefill hand-off give-ups,
 *     pooled-decode slot conflicts) persist between calls until their query resets
 *     them.  The decode entry points keep no other state.
 *   - Thread safety: every entry point may be called from any host thread; the
 *     per-device state above is guarded by its mutex.
 *
 * Return value: GDN_OK (0) on success, otherwise a GDN_ERR_* code; the
 * calling thread's gdn_last_error() then describes the failure.  Argument
 * validation happens before any device call, so invalid arguments are reported
 * without touching a GPU.
 *
 * Head dims: dk = dv = 128.  GQA: v-head h reads q-head h / (Hv/Hq) and k-head
 * h / (Hv/Hk); Hv must be a multiple of Hq and of Hk.
 * scale == 0 selects the default 1/sqrt(dk).
 */
#ifndef GDN_KERNEL_AMD_H
#define GDN_KERNEL_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t gdn_bf16; /* raw bf16 bits */

#define GDN_OK 0
#define GDN_ERR_INVALID_ARGUMENT 1 /* bad pointer, size, head ratio, dtype code */
#define GDN_ERR_UNSUPPORTED 2      /* valid request this build does not implement */
#define GDN_ERR_DEVICE 3           /* HIP launch / runtime error */

#define GDN_INDEX_INT32 0
#define GDN_INDEX_INT64 1

/* Largest head count (num_q_heads, num_k_heads, num_v_heads) the kernels address:
 * their per-chunk row offsets (up to 64 tokens x heads x 128 elements) are 32-bit.
 * Larger counts return GDN_ERR_UNSUPPORTED. */
#define GDN_MAX_HEADS 65536

/* Library version, as MAJOR*10000 + MINOR*100 + PATCH. */
int gdn_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* gdn_last_error(void);

/* Build id: 16 hex digits of SHA-256 over the headers, sources and compiler flags
 * the library was built from (gdn_kernel_amd.build.source_digest), so a built
 * library can be matched with its sources.  No reference counterpart. */
const char* gdn_build_id(void);

/*
 * Decode step, destination-passing.  Replaces the reference's TVM-FFI export
 * `kernel` = GDNDecodeKernel (solution/cuda/kernel.cu:101-113, exported at
 * :150), same argument order: q, k, v, state, A_log, a, dt_bias, b, scale,
 * output, new_state.
 *   q [B,1,Hq,128] bf16, k [B,1,Hk,128] bf16, v [B,1,Hv,128] bf16
 *   state     [B,Hv,128,128] fp32, or NULL for a zero initial state
 *             (the reference memsets new_state and aliases it, kernel.cu:135-139)
 *   A_log [Hv] fp32, a [B,1,Hv] bf16, dt_bias [Hv] fp32, b [B,1,Hv] bf16
 *   output    [B,1,Hv,128] bf16
 *   new_state [B,Hv,128,128] fp32; may be the same pointer as state (in place)
 */
int gdn_decode(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
               const float* state, const float* A_log, const gdn_bf16* a,
               const float* dt_bias, const gdn_bf16* b, double scale,
               gdn_bf16* output, float* new_state, int64_t batch,
               int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
               int32_t head_dim_k, int32_t head_dim_v, void* stream);

/* Validation of gdn_decode's arguments only; touches no device. */
int gdn_decode_check(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                     const float* state, const float* A_log, const gdn_bf16* a,
                     const float* dt_bias, const gdn_bf16* b, double scale,
                     gdn_bf16* output, float* new_state, int64_t batch,
                     int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                     int32_t head_dim_k, int32_t head_dim_v);

/*
 * Decode step over an indexed state pool, updated in place.  No reference
 * counterpart: it is the reference decode (kernel.cu:101-148) with the state
 * of batch row i read from and written back to pool slot state_indices[i].
 *   state_pool    [pool_slots,Hv,128,128] fp32 (read and written)
 *   state_indices [B] int32 device array; an index outside [0, pool_slots)
 *                 marks a padding row: its output is zero and no slot is touched.
 * A slot that two or more valid rows name is a conflict: updating it from both rows
 * would race.  The kernel detects it on the device before it touches any state
 * (each row's workgroups scan the B indices) and skips every such row like a padding
 * row (zero output, slot untouched); gdn_decode_pool_conflicts counts the skipped
 * rows.  Other arguments as gdn_decode.
 */
int gdn_decode_pooled(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                      float* state_pool, int64_t pool_slots,
                      const int32_t* state_indices, const float* A_log,
                      const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                      double scale, gdn_bf16* output, int64_t batch,
                      int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                      int32_t head_dim_k, int32_t head_dim_v, void* stream);

int gdn_decode_pooled_check(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                            float* state_pool, int64_t pool_slots,
                            const int32_t* state_indices, const float* A_log,
                            const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                            double scale, gdn_bf16* output, int64_t batch,
                            int32_t num_q_heads, int32_t num_k_heads,
                            int32_t num_v_heads, int32_t head_dim_k,
                            int32_t head_dim_v);

/*
 * Conflict report of gdn_decode_pooled.  No reference counterpart (the reference has
 * no pooled decode).  Synchronises the current device, stores in *count the number of
 * pooled rows skipped because another row of their batch named the same slot (since
 * the library was loaded, or since the last reset), and with reset != 0 clears it.
 */
int gdn_decode_pool_conflicts(uint64_t* count, int32_t reset);

/* Bytes of device memory the library holds on each device its code is loaded onto
 * (the scratch arrays and counters above), for memory accounting. */
int64_t gdn_static_device_bytes(void);

/*
 * Varlen chunked prefill (chunk 64), destination-passing.  Replaces the
 * reference's TVM-FFI export `kernel` = GDNPrefillKernel
 * (solution/cuda/kernel_prefill.cu:300-306, exported at :339), same argument
 * order: q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
 * new_state.
 *   q [T,Hq,128] bf16, k [T,Hk,128] bf16, v [T,Hv,128] bf16 (packed tokens)
 *   state     [N,Hv,128,128] fp32 initial states, or NULL for zeros
 *   A_log [Hv] fp32, a [T,Hv] bf16, dt_bias [Hv] fp32, b [T,Hv] bf16
 *   cu_seqlens [N+1] device array, GDN_INDEX_INT32 or GDN_INDEX_INT64
 *             (the reference takes int64, kernel_prefill.cu:46); sequence i is
 *             tokens [cu[i], cu[i+1]).  An empty sequence passes its initial
 *             state through.  Entries are clamped into [0, T] on the device,
 *             so malformed offsets cannot make the kernel read out of bounds.
 *   output    [T,Hv,128] bf16
 *   new_state [N,Hv,128,128] fp32 final states; may alias state.
 * Nothing is allocated per call.  A batch whose sequences average at least
 * GDN_PREFILL_DROPIN_TWO_KERNEL_TOKENS (1,024) tokens (total_tokens >= 1,024
 * num_seqs) and whose chains the launcher splits over
 * several workgroups (at most 64 (sequence, v-head) chains on 256 CUs) runs the
 * two-kernel path of gdn_prefill_with_workspace (each chunk prepared once) in a
 * scratch array the library holds on each device (GDN_PREFILL_DROPIN_SCRATCH_BYTES,
 * its own, not gdn_prefill_no_alloc's), when its chunk images fit:
 * gdn_prefill_workspace_size(num_seqs, total_tokens, Hv) bytes, 19,200 per 64-token
 * chunk and v-head of each sequence's ceil(total_tokens / 64) chunk slots, so with
 * one sequence and 32 v-heads up to 13,952 tokens (BASELINE's 4,096-token sequence
 * needs 37.5 MiB).  Larger batches run one kernel (one 16,384-token sequence: about
 * 8 % slower than two).  The results are the same bit for bit either way.  The library orders those launches on the device (each
 * waits, on its stream, for an event that the previous one records as it
 * completes), so calls on any streams stay correct; on a stream that is being
 * captured into a graph such a call runs one kernel instead.
 */
#define GDN_PREFILL_DROPIN_SCRATCH_BYTES (128LL << 20)
#define GDN_PREFILL_DROPIN_TWO_KERNEL_TOKENS 1024

int gdn_prefill(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                const float* state, const float* A_log, const gdn_bf16* a,
                const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                double scale, gdn_bf16* output, float* new_state,
                int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                int32_t head_dim_k, int32_t head_dim_v, void* stream);

int gdn_prefill_check(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                      const float* state, const float* A_log, const gdn_bf16* a,
                      const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                      int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                      double scale, gdn_bf16* output, float* new_state,
                      int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                      int32_t head_dim_k, int32_t head_dim_v);

/*
 * Prefill with a caller-owned device workspace.  No reference counterpart (the
 * reference allocates nothing and has no workspace argument); the Python
 * binding's `prefill_kernel_with_workspace` calls it.  Batches of few (sequence, head) chains (at most 64
 * on a 256-CU device) are split 4 or 8 ways across workgroups, each of which
 * would repeat the chunk preparation (T~, P and the gates).  With a workspace, the
 * preparation runs once per chunk in a first kernel, for all chunks in
 * parallel, and the state pass only copies it.
 *   gdn_prefill_workspace_size: bytes this path needs for num_seqs sequences,
 *     total_tokens tokens and num_v_heads v-heads on the current device;
 *     0 when gdn_prefill serves the batch with one kernel anyway (more chains,
 *     or more than 2 GiB of workspace).  Touches no device memory.
 *   gdn_prefill_with_workspace: gdn_prefill's arguments plus the workspace
 *     (16-byte aligned, at least the size above, and not shared with a launch
 *     that may run concurrently).  A NULL workspace, or a batch whose size is 0,
 *     runs gdn_prefill.  The results equal gdn_prefill's bit for bit (the same
 *     code prepares the chunks).
 */
int64_t gdn_prefill_workspace_size(int64_t num_seqs, int64_t total_tokens,
                                   int32_t num_v_heads);

int gdn_prefill_with_workspace(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                               const float* state, const float* A_log, const gdn_bf16* a,
                               const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                               int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                               double scale, gdn_bf16* output, float* new_state,
                               int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                               int32_t head_dim_k, int32_t head_dim_v, void* workspace,
                               int64_t workspace_bytes, void* stream);

/*
 * gdn_prefill_with_workspace for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference, which has no workspace.  Same
 * arguments and results as gdn_prefill (bit for bit); the chunk images of the
 * two-kernel path live in a scratch array that the library holds on each device
 * (GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES, allocated when the library's code is
 * loaded onto the device and kept until the process ends).  Nothing is allocated
 * per call.  A batch whose images need more than that (gdn_prefill_workspace_size
 * above it) returns GDN_ERR_INVALID_ARGUMENT; batches that gdn_prefill serves with
 * one kernel need no scratch.  Every call on a device shares that device's
 * scratch.  Calls on streams that are not being captured are ordered on the device
 * like gdn_prefill's (their own mutex and event), so eager calls on any streams stay
 * correct.  A call captured into a graph cannot wait for that event: its replays
 * must not overlap with any other call of gdn_prefill_no_alloc on the same GPU
 * (eager or replayed), or they race and give wrong results.
 */
#define GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES (64LL << 20)

int gdn_prefill_no_alloc(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v,
                         const float* state, const float* A_log, const gdn_bf16* a,
                         const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                         int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                         double scale, gdn_bf16* output, float* new_state,
                         int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                         int32_t head_dim_k, int32_t head_dim_v, void* stream);

/*
 * Failure report of the prefill kernels' hand-off waits.  No reference
 * counterpart: the reference prefill kernel synchronises with workgroup barriers
 * only (kernel_prefill.cu:149-161) and has no bounded wait that could fail.
 * Here the wavefronts of a prefill workgroup hand chunks to each other through
 * bounded waits (about 70 ms of polling).  A wait that gives up -- which only a
 * defect could cause -- lets the workgroup finish instead of hanging the GPU; the
 * workgroup then writes NaN to every output and final-state element it owns, and
 * each wavefront that gave up adds 1 to a counter on the device.
 * gdn_prefill_giveups synchronises the current device, stores that counter (the
 * give-ups since the library was loaded, or since the last reset) in *count, and
 * with reset != 0 clears it.  A launch that returned GDN_OK and left the counter
 * at 0 completed every hand-off.
 */
int gdn_prefill_giveups(uint64_t* count, int32_t reset);

#ifdef __cplusplus
}
#endif

#endif /* GDN_KERNEL_AMD_H */

// Internal launcher interface between the C-ABI layer (gdn_capi.cpp) and the
// kernel translation units.  Arguments here are already validated.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

struct DecodeArgs {
  const uint16_t* q;        // [B, Hq, 128] bf16
  const uint16_t* k;        // [B, Hk, 128] bf16
  const uint16_t* v;        // [B, Hv, 128] bf16
  const float* state;       // [B|slots, Hv, 128, 128]; null => zero initial state
  float* new_state;         // same layout; may alias state
  const float* A_log;       // [Hv]
  const uint16_t* a;        // [B, Hv] bf16
  const float* dt_bias;     // [Hv]
  const uint16_t* b;        // [B, Hv] bf16
  const int32_t* slots;     // pooled mode: state head block = slots[bi]; else null
  int64_t pool_slots;       // pooled mode: number of slots in the pool
  uint16_t* out;            // [B, Hv, 128] bf16
  float scale;
  int B, Hq, Hk, Hv;
};

struct PrefillArgs {
  const uint16_t* q;        // [T, Hq, 128] bf16
  const uint16_t* k;        // [T, Hk, 128] bf16
  const uint16_t* v;        // [T, Hv, 128] bf16
  const float* state;       // [N, Hv, 128, 128] initial states; null => zeros
  float* new_state;         // [N, Hv, 128, 128] final states; may alias state
  const float* A_log;       // [Hv]
  const uint16_t* a;        // [T, Hv] bf16
  const float* dt_bias;     // [Hv]
  const uint16_t* b;        // [T, Hv] bf16
  const void* cu_seqlens;   // [N + 1] int32 or int64
  int cu_is_64;             // 1 => int64 cu_seqlens
  uint16_t* out;            // [T, Hv, 128] bf16
  float scale;
  int64_t T;                // total packed tokens
  int N, Hq, Hk, Hv;
  // Testing hooks for the hand-off failure path (zero in production launches):
  int spin_limit;           // polls before a hand-off wait gives up; 0 => the default (~70 ms)
  int ready_chunks;         // > 0: producers signal "chunk ready" only for chunks < ready_chunks
  unsigned* aborts;         // non-null: +1 (device atomic) each time a wait gives up
  // Two-kernel path: workspace of prefill_workspace_bytes(...) bytes for the
  // prepared T~/P tiles; null (or a batch that the single kernel serves) => one kernel.
  uint16_t* tiles;
  int prep_chunks;          // set by the launcher: consecutive chunks per prep workgroup
};

// Workspace bytes of the two-kernel prefill path for these sizes on the current
// device, or 0 when the single kernel serves them (many chains, or a workspace
// above the cap).
int64_t prefill_workspace_bytes(int N, int64_t T, int Hv);

// Decode launch shapes (rows per wave x waves per workgroup x nontemporal state
// access), numbered 0 .. kDecodeVariants-1; variant < 0 picks by batch size.
constexpr int kDecodeVariants = 16;
hipError_t launch_decode(const DecodeArgs& args, hipStream_t stream, int variant = -1);

// The decode launch shape used for `heads` = B * Hv (b, v-head) pairs when no
// variant is requested, and the work-items one head takes in a variant (the grid
// is heads * decode_items_per_head(v) / block work-items).
int decode_pick_variant(int64_t heads);
int64_t decode_items_per_head(int variant);

// Rows of pooled decode launches on the current device that were skipped because
// another row of their batch named the same slot, since the library was loaded or
// the last reset; synchronises the device first.
hipError_t decode_pool_conflicts(uint64_t* count, bool reset);

// Work-items of a prefill main-kernel launch for this many (sequence, v-head)
// chains on the current device (the grid times the workgroup size of the variant
// the launcher picks).
int64_t prefill_work_items(int64_t chains);
// `done`, if not null, is recorded when the launch's last kernel completes (the
// two-kernel path only: callers that pass it have set args.tiles).
hipError_t launch_prefill(const PrefillArgs& args, hipStream_t stream, hipEvent_t done = nullptr);

// Bytes of the per-device scratch array of gdn_prefill_no_alloc, and its address
// on the current device (looked up on the first call per device).
constexpr int64_t kPrefillScratchBytes = int64_t(64) << 20;
hipError_t prefill_scratch(void** ptr);

// The drop-in gdn_prefill's launcher: launch_prefill, except that a batch of few
// chains whose sequences average at least kDropinTwoKernelTokens tokens runs the
// two-kernel path in a per-device scratch of the library (kPrefillDropinScratchBytes)
// when its images fit, ordered between launches by an event.
constexpr int64_t kPrefillDropinScratchBytes = int64_t(128) << 20;
constexpr int64_t kDropinTwoKernelTokens = 1024;
hipError_t launch_prefill_dropin(const PrefillArgs& args, hipStream_t stream);

// gdn_prefill_no_alloc's launcher: the two-kernel path (for batches that take it) in
// the kPrefillScratchBytes array; eager launches are ordered between each other by an
// event, like the drop-in's.  The caller has checked that the images fit.
hipError_t launch_prefill_no_alloc(const PrefillArgs& args, hipStream_t stream);

// Device memory the library holds on every device its code is loaded onto, from load
// until the process ends: the two prefill scratch arrays and the device counters.
int64_t prefill_static_device_bytes();
int64_t decode_static_device_bytes();

// Waves of prefill launches on the current device whose hand-off wait gave up,
// since the library was loaded or the last reset; synchronises the device first.
hipError_t prefill_giveups(uint64_t* count, bool reset);

}  // namespace gdn

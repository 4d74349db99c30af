// C-ABI entry points: argument validation (host only, no device calls) and
// dispatch to the kernel launchers.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/gdn_kernel_amd.h"
#include "../../include/gdn_kernel_amd_testing.h"
#include "gdn_launch.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return GDN_OK;
}

constexpr int kD = 128;
constexpr int64_t kMaxGrid = 0x7fffffff;
// A launch's grid times its workgroup size (work-items per dimension) must fit in
// 32 bits.
constexpr int64_t kMaxWorkItems = 0xffffffffLL;
static_assert(int64_t(64 + 16) * GDN_MAX_HEADS * 128 < (int64_t(1) << 31),
              "per-chunk row offsets of GDN_MAX_HEADS heads fit 32 bits");
static_assert(GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES == gdn::kPrefillScratchBytes,
              "the header's scratch size must match the library's");
static_assert(GDN_PREFILL_DROPIN_SCRATCH_BYTES == gdn::kPrefillDropinScratchBytes,
              "the header's drop-in scratch size must match the library's");
static_assert(GDN_PREFILL_DROPIN_TWO_KERNEL_TOKENS == gdn::kDropinTwoKernelTokens,
              "the header's drop-in two-kernel threshold must match the library's");

int check_heads(int32_t hq, int32_t hk, int32_t hv, int32_t dk, int32_t dv) {
  if (hq <= 0 || hk <= 0 || hv <= 0)
    return fail(GDN_ERR_INVALID_ARGUMENT, "head counts must be positive (Hq=%d Hk=%d Hv=%d)", hq, hk, hv);
  if (hv % hq != 0 || hv % hk != 0)
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "num_v_heads (%d) must be a multiple of num_q_heads (%d) and num_k_heads (%d)", hv, hq, hk);
  // Per-chunk row offsets in the kernels (up to 64 tokens x heads x 128 elements) are
  // 32-bit; num_q_heads and num_k_heads divide num_v_heads, so bounding it bounds all.
  if (hv > GDN_MAX_HEADS)
    return fail(GDN_ERR_UNSUPPORTED, "num_v_heads (%d) is above the %d heads the kernels address", hv,
                GDN_MAX_HEADS);
  if (dk <= 0 || dv <= 0)
    return fail(GDN_ERR_INVALID_ARGUMENT, "head dims must be positive (dk=%d dv=%d)", dk, dv);
  if (dk != kD || dv != kD)
    return fail(GDN_ERR_UNSUPPORTED, "only head_dim_k == head_dim_v == 128 is implemented (got %d, %d)", dk, dv);
  return GDN_OK;
}

int check_scale(double scale) {
  if (!std::isfinite(scale)) return fail(GDN_ERR_INVALID_ARGUMENT, "scale must be finite");
  return GDN_OK;
}

float resolve_scale(double scale) {
  return scale == 0.0 ? 1.0f / std::sqrt(float(kD)) : float(scale);
}

// new_state may equal state (in place) but must not partially overlap it.
int check_alias(const void* in, const void* out, int64_t bytes, const char* what) {
  if (!in || !out || in == out || bytes <= 0) return GDN_OK;
  const char* a = static_cast<const char*>(in);
  const char* b = static_cast<const char*>(out);
  if (a < b + bytes && b < a + bytes)
    return fail(GDN_ERR_INVALID_ARGUMENT, "%s partially overlaps its input (only exact aliasing is allowed)", what);
  return GDN_OK;
}

#define GDN_TRY(expr)            \
  do {                           \
    const int rc_ = (expr);      \
    if (rc_ != GDN_OK) return rc_; \
  } while (0)

int device_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(GDN_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// The decode grid of `variant` (or of the launcher's own pick, variant < 0) for
// batch * num_v_heads heads must fit: work-items in 32 bits (and the batch in an int).
int check_decode_launch(int64_t batch, int32_t num_v_heads, int variant) {
  const int64_t heads = batch * num_v_heads;
  const int vi = variant >= 0 ? variant : gdn::decode_pick_variant(heads);
  const int64_t per_head = gdn::decode_items_per_head(vi);
  if (batch > kMaxGrid || heads > kMaxWorkItems / per_head)
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "batch * num_v_heads = %lld is too large: the launch would need %lld work-items per "
                "head, at most %lld in total",
                (long long)heads, (long long)per_head, (long long)kMaxWorkItems);
  return GDN_OK;
}

int decode_check_impl(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                      const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                      double scale, gdn_bf16* output, float* new_state, int64_t batch, int32_t num_q_heads,
                      int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v,
                      int variant) {
  if (batch < 0) return fail(GDN_ERR_INVALID_ARGUMENT, "batch must be >= 0 (got %lld)", (long long)batch);
  GDN_TRY(check_heads(num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v));
  GDN_TRY(check_scale(scale));
  if (batch == 0) return ok();
  if (!q || !k || !v || !A_log || !a || !dt_bias || !b || !output || !new_state)
    return fail(GDN_ERR_INVALID_ARGUMENT, "null tensor pointer (only state may be null)");
  GDN_TRY(check_decode_launch(batch, num_v_heads, variant));
  GDN_TRY(check_alias(state, new_state, batch * num_v_heads * int64_t(kD) * kD * 4, "new_state"));
  return ok();
}

int decode_pooled_check_impl(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, float* state_pool,
                             int64_t pool_slots, const int32_t* state_indices, const float* A_log,
                             const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, double scale,
                             gdn_bf16* output, int64_t batch, int32_t num_q_heads, int32_t num_k_heads,
                             int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v, int variant) {
  if (batch < 0) return fail(GDN_ERR_INVALID_ARGUMENT, "batch must be >= 0 (got %lld)", (long long)batch);
  if (pool_slots <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "pool_slots must be > 0 (got %lld)", (long long)pool_slots);
  GDN_TRY(check_heads(num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v));
  GDN_TRY(check_scale(scale));
  if (batch == 0) return ok();
  if (!q || !k || !v || !state_pool || !state_indices || !A_log || !a || !dt_bias || !b || !output)
    return fail(GDN_ERR_INVALID_ARGUMENT, "null tensor pointer");
  GDN_TRY(check_decode_launch(batch, num_v_heads, variant));
  return ok();
}

}  // namespace

extern "C" {

int gdn_version(void) { return 100; }

const char* gdn_last_error(void) { return g_err; }

#ifndef GDN_BUILD_ID
#define GDN_BUILD_ID "unknown"
#endif
const char* gdn_build_id(void) { return GDN_BUILD_ID; }

int gdn_decode_check(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                     const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                     double scale, gdn_bf16* output, float* new_state, int64_t batch, int32_t num_q_heads,
                     int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v) {
  return decode_check_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch, num_q_heads,
                           num_k_heads, num_v_heads, head_dim_k, head_dim_v, -1);
}

int gdn_decode_pooled_check(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, float* state_pool,
                            int64_t pool_slots, const int32_t* state_indices, const float* A_log,
                            const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, double scale,
                            gdn_bf16* output, int64_t batch, int32_t num_q_heads, int32_t num_k_heads,
                            int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v) {
  return decode_pooled_check_impl(q, k, v, state_pool, pool_slots, state_indices, A_log, a, dt_bias, b, scale,
                                  output, batch, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v,
                                  -1);
}

int gdn_prefill_check(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                      const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                      const void* cu_seqlens, int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                      double scale, gdn_bf16* output, float* new_state, int32_t num_q_heads, int32_t num_k_heads,
                      int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v) {
  if (num_seqs < 0) return fail(GDN_ERR_INVALID_ARGUMENT, "num_seqs must be >= 0 (got %lld)", (long long)num_seqs);
  if (total_tokens < 0)
    return fail(GDN_ERR_INVALID_ARGUMENT, "total_tokens must be >= 0 (got %lld)", (long long)total_tokens);
  if (total_tokens > kMaxGrid)
    return fail(GDN_ERR_INVALID_ARGUMENT, "total_tokens too large (%lld)", (long long)total_tokens);
  if (cu_seqlens_dtype != GDN_INDEX_INT32 && cu_seqlens_dtype != GDN_INDEX_INT64)
    return fail(GDN_ERR_INVALID_ARGUMENT, "cu_seqlens_dtype must be GDN_INDEX_INT32 or GDN_INDEX_INT64 (got %d)",
                cu_seqlens_dtype);
  GDN_TRY(check_heads(num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v));
  GDN_TRY(check_scale(scale));
  if (num_seqs == 0) return ok();
  if (num_seqs > kMaxGrid || num_seqs * num_v_heads > kMaxGrid ||
      gdn::prefill_work_items(num_seqs * num_v_heads) > kMaxWorkItems)
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "num_seqs * num_v_heads = %lld is too large: the launch would exceed %lld work-items",
                (long long)(num_seqs * num_v_heads), (long long)kMaxWorkItems);
  if (!cu_seqlens || !A_log || !dt_bias || !new_state)
    return fail(GDN_ERR_INVALID_ARGUMENT, "null tensor pointer (only state may be null)");
  if (total_tokens > 0 && (!q || !k || !v || !a || !b || !output))
    return fail(GDN_ERR_INVALID_ARGUMENT, "null tensor pointer (only state may be null)");
  GDN_TRY(check_alias(state, new_state, num_seqs * num_v_heads * int64_t(kD) * kD * 4, "new_state"));
  return ok();
}

}  // extern "C"

namespace {

int decode_impl(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, double scale,
                gdn_bf16* output, float* new_state, int64_t batch, int32_t num_q_heads, int32_t num_k_heads,
                int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v, int variant, void* stream) {
  GDN_TRY(decode_check_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch, num_q_heads,
                            num_k_heads, num_v_heads, head_dim_k, head_dim_v, variant));
  if (batch == 0) return ok();
  gdn::DecodeArgs args{};
  args.q = q; args.k = k; args.v = v;
  args.state = state; args.new_state = new_state;
  args.A_log = A_log; args.a = a; args.dt_bias = dt_bias; args.b = b;
  args.slots = nullptr; args.pool_slots = 0;
  args.out = output;
  args.scale = resolve_scale(scale);
  args.B = int(batch); args.Hq = num_q_heads; args.Hk = num_k_heads; args.Hv = num_v_heads;
  return device_status(gdn::launch_decode(args, static_cast<hipStream_t>(stream), variant), "gdn_decode launch");
}

int decode_pooled_impl(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, float* state_pool,
                       int64_t pool_slots, const int32_t* state_indices, const float* A_log, const gdn_bf16* a,
                       const float* dt_bias, const gdn_bf16* b, double scale, gdn_bf16* output, int64_t batch,
                       int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k,
                       int32_t head_dim_v, int variant, void* stream) {
  GDN_TRY(decode_pooled_check_impl(q, k, v, state_pool, pool_slots, state_indices, A_log, a, dt_bias, b, scale,
                                   output, batch, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v,
                                   variant));
  if (batch == 0) return ok();
  gdn::DecodeArgs args{};
  args.q = q; args.k = k; args.v = v;
  args.state = state_pool; args.new_state = state_pool;
  args.A_log = A_log; args.a = a; args.dt_bias = dt_bias; args.b = b;
  args.slots = state_indices; args.pool_slots = pool_slots;
  args.out = output;
  args.scale = resolve_scale(scale);
  args.B = int(batch); args.Hq = num_q_heads; args.Hk = num_k_heads; args.Hv = num_v_heads;
  return device_status(gdn::launch_decode(args, static_cast<hipStream_t>(stream), variant),
                       "gdn_decode_pooled launch");
}

// Launcher of a prefill call: launch_prefill (optionally with a caller workspace),
// the drop-in's (its own ordered scratch for batches of long sequences) or
// gdn_prefill_no_alloc's (the library's ordered scratch).
enum class PrefillPath { kPlain, kDropin, kNoAlloc };

int prefill_impl(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state, const float* A_log,
                 const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                 int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens, double scale, gdn_bf16* output,
                 float* new_state, int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                 int32_t head_dim_k, int32_t head_dim_v, int32_t spin_limit, int32_t ready_chunks,
                 uint32_t* aborts, void* workspace, int64_t workspace_bytes, void* stream,
                 PrefillPath path = PrefillPath::kPlain) {
  GDN_TRY(gdn_prefill_check(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_dtype, num_seqs,
                            total_tokens, scale, output, new_state, num_q_heads, num_k_heads, num_v_heads,
                            head_dim_k, head_dim_v));
  uint16_t* tiles = nullptr;
  if (workspace != nullptr) {
    const int64_t need = gdn::prefill_workspace_bytes(int(num_seqs), total_tokens, num_v_heads);
    if (need > 0) {
      if (workspace_bytes < need)
        return fail(GDN_ERR_INVALID_ARGUMENT, "workspace_bytes is %lld, this batch needs %lld",
                    static_cast<long long>(workspace_bytes), static_cast<long long>(need));
      if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
      tiles = static_cast<uint16_t*>(workspace);
    }
  }
  if (num_seqs == 0) return ok();
  gdn::PrefillArgs args{};
  args.tiles = tiles;
  args.spin_limit = spin_limit;
  args.ready_chunks = ready_chunks;
  args.aborts = aborts;
  args.q = q; args.k = k; args.v = v;
  args.state = state; args.new_state = new_state;
  args.A_log = A_log; args.a = a; args.dt_bias = dt_bias; args.b = b;
  args.cu_seqlens = cu_seqlens; args.cu_is_64 = cu_seqlens_dtype == GDN_INDEX_INT64;
  args.out = output;
  args.scale = resolve_scale(scale);
  args.T = total_tokens;
  args.N = int(num_seqs); args.Hq = num_q_heads; args.Hk = num_k_heads; args.Hv = num_v_heads;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e = path == PrefillPath::kDropin   ? gdn::launch_prefill_dropin(args, st)
                       : path == PrefillPath::kNoAlloc ? gdn::launch_prefill_no_alloc(args, st)
                                                       : gdn::launch_prefill(args, st);
  return device_status(e, "gdn_prefill launch");
}

int check_variant(int32_t variant) {
  if (variant < 0 || variant >= gdn::kDecodeVariants)
    return fail(GDN_ERR_INVALID_ARGUMENT, "variant must be in [0, %d) (got %d)", gdn::kDecodeVariants, variant);
  return ok();
}

}  // namespace

extern "C" {

int gdn_decode(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
               const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, double scale,
               gdn_bf16* output, float* new_state, int64_t batch, int32_t num_q_heads, int32_t num_k_heads,
               int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v, void* stream) {
  return decode_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch, num_q_heads,
                     num_k_heads, num_v_heads, head_dim_k, head_dim_v, -1, stream);
}

int gdn_decode_pooled(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, float* state_pool,
                      int64_t pool_slots, const int32_t* state_indices, const float* A_log, const gdn_bf16* a,
                      const float* dt_bias, const gdn_bf16* b, double scale, gdn_bf16* output, int64_t batch,
                      int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k,
                      int32_t head_dim_v, void* stream) {
  return decode_pooled_impl(q, k, v, state_pool, pool_slots, state_indices, A_log, a, dt_bias, b, scale, output,
                            batch, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v, -1, stream);
}

int gdn_prefill(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state, const float* A_log,
                const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, const void* cu_seqlens,
                int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens, double scale, gdn_bf16* output,
                float* new_state, int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads,
                int32_t head_dim_k, int32_t head_dim_v, void* stream) {
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_dtype, num_seqs, total_tokens,
                      scale, output, new_state, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v, 0, 0,
                      nullptr, nullptr, 0, stream, PrefillPath::kDropin);
}

int64_t gdn_prefill_workspace_size(int64_t num_seqs, int64_t total_tokens, int32_t num_v_heads) {
  if (num_seqs <= 0 || num_seqs > INT32_MAX || total_tokens <= 0 || num_v_heads <= 0) return 0;
  return gdn::prefill_workspace_bytes(int(num_seqs), total_tokens, num_v_heads);
}

int gdn_prefill_with_workspace(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                               const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                               const void* cu_seqlens, int32_t cu_seqlens_dtype, int64_t num_seqs,
                               int64_t total_tokens, double scale, gdn_bf16* output, float* new_state,
                               int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k,
                               int32_t head_dim_v, void* workspace, int64_t workspace_bytes, void* stream) {
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_dtype, num_seqs, total_tokens,
                      scale, output, new_state, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v, 0, 0,
                      nullptr, workspace, workspace_bytes, stream);
}

int gdn_prefill_no_alloc(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                         const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                         const void* cu_seqlens, int32_t cu_seqlens_dtype, int64_t num_seqs, int64_t total_tokens,
                         double scale, gdn_bf16* output, float* new_state, int32_t num_q_heads,
                         int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v,
                         void* stream) {
  GDN_TRY(gdn_prefill_check(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_dtype, num_seqs,
                            total_tokens, scale, output, new_state, num_q_heads, num_k_heads, num_v_heads,
                            head_dim_k, head_dim_v));
  const int64_t need = num_seqs > 0 ? gdn::prefill_workspace_bytes(int(num_seqs), total_tokens, num_v_heads) : 0;
  if (need > gdn::kPrefillScratchBytes)
    return fail(GDN_ERR_INVALID_ARGUMENT,
                "this batch needs %lld bytes of chunk images, more than the %lld-byte scratch of "
                "gdn_prefill_no_alloc; use gdn_prefill_with_workspace (or gdn_prefill)",
                static_cast<long long>(need), static_cast<long long>(gdn::kPrefillScratchBytes));
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_dtype, num_seqs, total_tokens,
                      scale, output, new_state, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v, 0, 0,
                      nullptr, nullptr, 0, stream, PrefillPath::kNoAlloc);
}

int64_t gdn_static_device_bytes(void) {
  return gdn::prefill_static_device_bytes() + gdn::decode_static_device_bytes();
}

int gdn_prefill_giveups(uint64_t* count, int32_t reset) {
  if (!count) return fail(GDN_ERR_INVALID_ARGUMENT, "count must not be null");
  return device_status(gdn::prefill_giveups(count, reset != 0), "gdn_prefill_giveups");
}

int gdn_decode_pool_conflicts(uint64_t* count, int32_t reset) {
  if (!count) return fail(GDN_ERR_INVALID_ARGUMENT, "count must not be null");
  return device_status(gdn::decode_pool_conflicts(count, reset != 0), "gdn_decode_pool_conflicts");
}

int gdn_decode_num_variants(void) { return gdn::kDecodeVariants; }

int gdn_decode_with_variant(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                            const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                            double scale, gdn_bf16* output, float* new_state, int64_t batch, int32_t num_q_heads,
                            int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v,
                            int32_t variant, void* stream) {
  GDN_TRY(check_variant(variant));
  return decode_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch, num_q_heads,
                     num_k_heads, num_v_heads, head_dim_k, head_dim_v, variant, stream);
}

int gdn_decode_pooled_with_variant(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, float* state_pool,
                                   int64_t pool_slots, const int32_t* state_indices, const float* A_log,
                                   const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b, double scale,
                                   gdn_bf16* output, int64_t batch, int32_t num_q_heads, int32_t num_k_heads,
                                   int32_t num_v_heads, int32_t head_dim_k, int32_t head_dim_v, int32_t variant,
                                   void* stream) {
  GDN_TRY(check_variant(variant));
  return decode_pooled_impl(q, k, v, state_pool, pool_slots, state_indices, A_log, a, dt_bias, b, scale, output,
                            batch, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v, variant, stream);
}

int gdn_prefill_fault_injection(const gdn_bf16* q, const gdn_bf16* k, const gdn_bf16* v, const float* state,
                                const float* A_log, const gdn_bf16* a, const float* dt_bias, const gdn_bf16* b,
                                const void* cu_seqlens, int32_t cu_seqlens_dtype, int64_t num_seqs,
                                int64_t total_tokens, double scale, gdn_bf16* output, float* new_state,
                                int32_t num_q_heads, int32_t num_k_heads, int32_t num_v_heads, int32_t head_dim_k,
                                int32_t head_dim_v, int32_t spin_limit, int32_t ready_chunks, uint32_t* aborts,
                                void* stream) {
  if (spin_limit < 0 || ready_chunks < 0)
    return fail(GDN_ERR_INVALID_ARGUMENT, "spin_limit and ready_chunks must be >= 0 (got %d, %d)", spin_limit,
                ready_chunks);
  return prefill_impl(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_dtype, num_seqs, total_tokens,
                      scale, output, new_state, num_q_heads, num_k_heads, num_v_heads, head_dim_k, head_dim_v,
                      spin_limit, ready_chunks, aborts, nullptr, 0, stream);
}

}  // extern "C"

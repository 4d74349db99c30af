// GDN decode step (T = 1) for gfx950: one pass over each head's fp32 state.
//
// Math per (batch b, v-head h), state S[v][k] (k contiguous), following the
// reference definition (design.md:166-226) in the single-pass form the
// reference kernel uses (kernel.cu:59-92):
//   g = exp(-exp(A_log) softplus(a + dt_bias)),  beta = sigmoid(b)
//   s_v   = g * S[v, :]                    (decayed row)
//   kv_v  = s_v . k,  qv_v = s_v . q       (two 128-long dots per row)
//   d_v   = beta (v_v - kv_v)
//   S'[v] = s_v + d_v k                    (rank-1 delta write)
//   o_v   = scale (qv_v + d_v (q . k))     (= scale * S'[v] . q)
//
// Data movement: the state is the only large operand (64 KiB per head).  Each
// wavefront owns RPW consecutive rows of one head.  Lane l holds columns
// 4*(l%32) .. +3 of rows 2j + l/32 (j < RPW/2), so every load instruction of a
// wave reads 1 KiB of contiguous state with 16-byte lanes.  All RPW/2 loads are
// issued before any arithmetic.  Rows are independent, so there is no LDS and no
// barrier: the dot products are reduced across the 32 lanes that share a row with
// DPP + ds_swizzle.  Each element is read and then written by the same lane, so
// new_state may alias state (in-place update).
#include "gdn_common.hpp"
#include "gdn_launch.hpp"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Rows of pooled decode launches on this device skipped because another row of the
// same batch named their slot, since the library was loaded or the count was last
// reset; read by decode_pool_conflicts.
__device__ unsigned long long gdn_decode_pool_conflict_count;

template <bool NT>
__device__ __forceinline__ float4 load_state(const float* p) {
  f32x4 v;
  if constexpr (NT) {
    v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  } else {
    v = *reinterpret_cast<const f32x4*>(p);
  }
  return make_float4(v[0], v[1], v[2], v[3]);
}

template <bool NT>
__device__ __forceinline__ void store_state(float* p, float4 x) {
  const f32x4 v = {x.x, x.y, x.z, x.w};
  if constexpr (NT) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
  } else {
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

// Whether a row other than `bi` of the batch's B slot indices names `slot`.  The
// WAVES waves of a workgroup (all on the same batch row) each scan an interleaved
// share of the indices, four 64-index blocks per pass, and OR their verdicts
// through LDS.  Ends with a workgroup barrier when WAVES > 1.
template <int WAVES>
__device__ __forceinline__ bool slot_named_elsewhere(const int32_t* slots, int B, int bi, int slot, int lane,
                                                     int wave) {
  constexpr int STEP = 64 * WAVES;
  bool hit = false;
  for (int i0 = 64 * wave; i0 < B; i0 += 4 * STEP) {
    int s[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * STEP + lane;
      s[u] = i < B ? slots[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) hit |= s[u] == slot && i0 + u * STEP + lane != bi;
  }
  const bool any = __builtin_amdgcn_ballot_w64(hit) != 0;
  if constexpr (WAVES == 1) {
    return any;
  } else {
    __shared__ int wave_hit[WAVES];
    if (lane == 0) wave_hit[wave] = any;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) r |= wave_hit[w];
    return r != 0;
  }
}

// RPW rows per wave, WAVES waves per workgroup; a workgroup covers RPW*WAVES
// rows of one head and 128 / (RPW*WAVES) workgroups cover one head.
template <int RPW, int WAVES, bool HAS_STATE, bool POOLED, bool NT>
__global__ __launch_bounds__(64 * WAVES) void gdn_decode_kernel(DecodeArgs p) {
  constexpr int D = kHeadDim;
  constexpr int NL = RPW / 2;
  constexpr int ROWS_PER_WG = RPW * WAVES;
  constexpr int WG_PER_HEAD = D / ROWS_PER_WG;
  static_assert(RPW % 2 == 0 && RPW <= 64 && D % ROWS_PER_WG == 0, "bad tiling");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = lane >> 5;
  const int col = (lane & 31) * 4;

  int blk = blockIdx.x;
  const int rblk = blk % WG_PER_HEAD;
  blk /= WG_PER_HEAD;
  const int h = blk % p.Hv;
  const int bi = blk / p.Hv;
  const int row0 = rblk * ROWS_PER_WG + wave * RPW;

  const int64_t head = int64_t(bi) * p.Hv + h;     // index of (b, h) in v/a/b/out
  uint16_t* outp = p.out + head * D + row0;

  int64_t shead = head;                             // index of the state block
  if constexpr (POOLED) {
    const int64_t slot = p.slots[bi];
    if (slot < 0 || slot >= p.pool_slots) {         // padding slot: zero output, no state
      if (lane < RPW) outp[lane] = 0;
      return;
    }
    // A slot that two rows of the batch name would be updated by both at once: such
    // rows are skipped like padding (zero output, slot untouched), decided before any
    // state access, and the first wave of each counts its row once.
    if (slot_named_elsewhere<WAVES>(p.slots, p.B, bi, int(slot), lane, wave)) {
      if (lane < RPW) outp[lane] = 0;
      if (h == 0 && row0 == 0 && lane == 0)
        __hip_atomic_fetch_add(&gdn_decode_pool_conflict_count, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    shead = slot * p.Hv + h;
  }

  // Gate and beta (every lane computes the same scalars).
  const float g = expf(log_gate(p.A_log[h], bf16_to_f32(p.a[head]), p.dt_bias[h]));
  const float beta = sigmoidf_(bf16_to_f32(p.b[head]));

  // This lane's 4 columns of q and k.
  const int hq = h / (p.Hv / p.Hq);
  const int hk = h / (p.Hv / p.Hk);
  const uint2 qw = *reinterpret_cast<const uint2*>(p.q + (int64_t(bi) * p.Hq + hq) * D + col);
  const uint2 kw = *reinterpret_cast<const uint2*>(p.k + (int64_t(bi) * p.Hk + hk) * D + col);
  const float q0 = __uint_as_float(qw.x << 16), q1 = __uint_as_float(qw.x & 0xffff0000u);
  const float q2 = __uint_as_float(qw.y << 16), q3 = __uint_as_float(qw.y & 0xffff0000u);
  const float k0 = __uint_as_float(kw.x << 16), k1 = __uint_as_float(kw.x & 0xffff0000u);
  const float k2 = __uint_as_float(kw.y << 16), k3 = __uint_as_float(kw.y & 0xffff0000u);

  // Issue every state load of this wave before any arithmetic.
  const int64_t sbase = (shead * D + row0 + half) * D + col;
  float4 s[NL];
  if constexpr (HAS_STATE) {
#pragma unroll
    for (int j = 0; j < NL; ++j) s[j] = load_state<NT>(p.state + sbase + int64_t(2 * j) * D);
  } else {
#pragma unroll
    for (int j = 0; j < NL; ++j) s[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const float vmine = lane < RPW ? bf16_to_f32(p.v[head * D + row0 + lane]) : 0.0f;
  const float qdotk = sum32(q0 * k0 + q1 * k1 + q2 * k2 + q3 * k3);

  float myout = 0.0f;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    float4 t = s[j];
    t.x *= g; t.y *= g; t.z *= g; t.w *= g;
    float kv = t.x * k0 + t.y * k1 + t.z * k2 + t.w * k3;
    float qv = t.x * q0 + t.y * q1 + t.z * q2 + t.w * q3;
    kv = sum32(kv);
    qv = sum32(qv);
    const float v0 = readlane_f(vmine, 2 * j);
    const float v1 = readlane_f(vmine, 2 * j + 1);
    const float delta = beta * ((half ? v1 : v0) - kv);
    t.x += k0 * delta; t.y += k1 * delta; t.z += k2 * delta; t.w += k3 * delta;
    store_state<NT>(p.new_state + sbase + int64_t(2 * j) * D, t);
    const float o = p.scale * (qv + delta * qdotk);
    if ((lane & 31) == j) myout = o;
  }
  if ((lane & 31) < NL) outp[2 * (lane & 31) + half] = f32_to_bf16(myout);
}

namespace {

// Launch shapes (rows per wave, waves per workgroup, nontemporal state access),
// numbered as the variant argument of launch_decode.
#define GDN_DECODE_VARIANTS(X)                                                              \
  X(0, 16, 4, true) X(1, 8, 4, true) X(2, 4, 4, true) X(3, 2, 4, true) X(4, 8, 2, true)    \
  X(5, 4, 2, true) X(6, 16, 2, true) X(7, 32, 4, true) X(8, 8, 1, true) X(9, 4, 1, true)   \
  X(10, 16, 4, false) X(11, 8, 4, false) X(12, 4, 4, false) X(13, 2, 2, true)              \
  X(14, 16, 1, true) X(15, 2, 1, true)
static_assert(kDecodeVariants == 16, "the variant table has 16 entries");

template <int RPW, int WAVES, bool NT>
hipError_t launch_variant(const DecodeArgs& a, hipStream_t stream) {
  const int64_t heads = int64_t(a.B) * a.Hv;
  const int64_t grid = heads * (kHeadDim / (RPW * WAVES));
  const dim3 block(64 * WAVES);
  if (a.slots) {
    hipLaunchKernelGGL((gdn_decode_kernel<RPW, WAVES, true, true, NT>), dim3(grid), block, 0, stream, a);
  } else if (a.state) {
    hipLaunchKernelGGL((gdn_decode_kernel<RPW, WAVES, true, false, NT>), dim3(grid), block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((gdn_decode_kernel<RPW, WAVES, false, false, NT>), dim3(grid), block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace

int decode_pick_variant(int64_t heads) {
  // Measured on MI355X (B=64 and pooled B=512, cold cache): 8 rows per wave,
  // 4 waves, nontemporal state traffic is fastest; small batches use one-wave
  // workgroups so that more CUs get work.
  return heads >= 128 ? 1 : 8;
}

int64_t decode_items_per_head(int variant) {
  switch (variant) {
#define GDN_ITEMS(I, R, W, NT) \
  case I:                      \
    return kHeadDim / (R) * 64;
    GDN_DECODE_VARIANTS(GDN_ITEMS)
#undef GDN_ITEMS
    default:
      return kHeadDim / 16 * 64;
  }
}

int64_t decode_static_device_bytes() { return int64_t(sizeof(gdn_decode_pool_conflict_count)); }

hipError_t decode_pool_conflicts(uint64_t* count, bool reset) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  unsigned long long v = 0;
  e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(gdn_decode_pool_conflict_count), sizeof(v));
  if (e != hipSuccess) return e;
  *count = v;
  if (reset) {
    const unsigned long long z = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(gdn_decode_pool_conflict_count), &z, sizeof(z));
  }
  return e;
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream, int variant) {
  int vi = variant;
  if (vi < 0 || vi >= kDecodeVariants) vi = decode_pick_variant(int64_t(a.B) * a.Hv);
  switch (vi) {
#define GDN_CASE(I, R, W, NT) \
  case I:                     \
    return launch_variant<R, W, NT>(a, stream);
    GDN_DECODE_VARIANTS(GDN_CASE)
#undef GDN_CASE
    default:
      return launch_variant<16, 4, true>(a, stream);
  }
}

}  // namespace gdn

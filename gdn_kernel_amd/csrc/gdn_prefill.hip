// GDN varlen chunked prefill for gfx950 (chunk C = 64, dk = dv = 128).
//
// One workgroup of 4 wavefronts walks the chunks of one (sequence, v-head)
// chain.  The fp32 state never leaves the register file between chunks: wave w
// owns state rows v in [32w, 32w+32) as MFMA accumulators (16x16 tiles of S^T,
// lane = (k-group g = lane/16, column n = lane%16) holding S[v][k..k+3]).
//
// Per chunk (positions >= clen are zero-padded: K = Q = V = 0, beta = 0 and
// log-gate 0, as kernel_prefill.cu:102-114, 125-132 pads them):
//   gamma = inclusive cumsum of the log gates, beta = sigmoid(b)   (a1, :101-122)
//   N[i][j] = beta_i e^{gamma_i - gamma_j} k_i.k_j   (i > j)       (:134-146, sign folded)
//   P[i][j] = e^{gamma_i - gamma_j} q_i.k_j          (j <= i)       (:165-185)
//   T~ = (I + N)^-1                                   (:148-163)
//   X  = K S^T                                        (retrieval from the chunk-start state)
//   Y  = beta (V - e^gamma X)
//   v_new = T~ Y          (= T~(beta V) - T~(beta e^gamma K) S^T = U - W S^T, :187-195, 236-271)
//   o  = scale (e^gamma Q S^T + P v_new)              (:216-234, 273-283)
//   S  = e^{gamma_last} S + (d v_new)^T K,  d_c = e^{gamma_last - gamma_c}   (:197-202, 286-293)
//
// Precision: q/k/v are exact bf16 MFMA operands.  Operands that are fp32 values
// (S, Y, T~, d*v_new) are split into bf16 hi + lo pairs so that the products
// that feed the state carry ~16 mantissa bits; fp32 accumulation throughout.
// The output-only product P v_new uses the bf16 hi parts alone.
//
// MFMA operand convention (v_mfma_f32_16x16x32_bf16): lane l supplies row/col
// l%16 and 8 contraction elements chosen by g = l/16.  This file pairs A and B
// consistently with contraction index kappa(g, s) = 4g + s (s < 4) and
// 16 + 4g + (s - 4) (s >= 4) inside each 32-wide block, which is exactly what an
// accumulator pair (two 16x16 tiles stacked along the contraction dim) holds.
// So accumulators become B operands without leaving registers, and LDS tiles
// are stored with their contraction columns permuted (perm32) so an A fragment is
// one 16-byte LDS read.
#include "gdn_common.hpp"
#include "gdn_launch.hpp"

namespace gdn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int C = 64;       // chunk length
constexpr int D = kHeadDim; // 128
constexpr int KSTR = 136;   // bf16 row stride of the K / Q chunk tiles
constexpr int TSTR = 72;    // bf16 row stride of 64-wide operand tiles (K^T, T~, P)
constexpr int FSTR = 68;    // fp32 row stride of the 64x64 solve matrices
constexpr int NTHREADS = 256;

struct __align__(16) PrefillSmem {
  uint16_t K[C * KSTR];     // K chunk [c][perm(k)]
  uint16_t Q[C * KSTR];     // Q chunk [c][perm(k)]
  uint16_t V[C * KSTR];     // V chunk [c][v]
  uint16_t O[C * KSTR];     // output tile [c][v], staged for 16-byte stores
  uint16_t Kt[D * TSTR];    // K^T     [k][perm(c)]
  uint16_t Th[C * TSTR];    // T~ hi   [c][perm(j)]
  uint16_t Tl[C * TSTR];    // T~ lo   [c][perm(j)]
  uint16_t P[C * TSTR];     // P (bf16)[c][perm(j)]
  float N[C * FSTR];        // N (fp32, strictly lower)
  float X[C * FSTR];        // T~ (fp32) and solve scratch in its upper blocks
  float gam[C];             // gamma_c (inclusive cumsum of the log gates)
  float bet[C];             // beta_c
  float eg[C];              // e^{gamma_c}
  float dd[C];              // e^{gamma_last - gamma_c}
};

constexpr float kLog2e = 1.4426950408889634f;

// e^{x} for x <= 0 via the hardware exp2 (v_exp_f32).
__device__ __forceinline__ float exp_le0(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ f32x4 mfma(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Position of contraction index r (0..31) inside a 32-wide permuted block.
__device__ __forceinline__ int perm32(int r) { return ((r & 15) >> 2) * 8 + ((r >> 4) << 2) + (r & 3); }
__device__ __forceinline__ int perm(int x) { return (x & ~31) + perm32(x & 31); }

// A fragment: rows row0 + lane%16, contraction block ks (32 wide), from a tile
// stored with permuted columns.
__device__ __forceinline__ uint4 frag(const uint16_t* tile, int stride, int row0, int ks, int lane) {
  return *reinterpret_cast<const uint4*>(tile + (row0 + (lane & 15)) * stride + 32 * ks + 8 * (lane >> 4));
}

// B fragment (bf16 hi parts) from two accumulator tiles stacked along the
// contraction dim.
__device__ __forceinline__ uint4 pack_hi(const f32x4& t0, const f32x4& t1) {
  return uint4{pack_bf16x2(t0[0], t0[1]), pack_bf16x2(t0[2], t0[3]), pack_bf16x2(t1[0], t1[1]),
               pack_bf16x2(t1[2], t1[3])};
}
// bf16 lo parts x - hi(x) (exact in fp32), rounded to bf16, given the hi words.
__device__ __forceinline__ uint32_t lo_word(float a, float b, uint32_t hi) {
  return pack_bf16x2(a - bf16lo_f32(hi), b - bf16hi_f32(hi));
}
__device__ __forceinline__ void split_pack(const f32x4& t0, const f32x4& t1, uint4& hi, uint4& lo) {
  hi = pack_hi(t0, t1);
  lo = uint4{lo_word(t0[0], t0[1], hi.x), lo_word(t0[2], t0[3], hi.y), lo_word(t1[0], t1[1], hi.z),
             lo_word(t1[2], t1[3], hi.w)};
}

__device__ __forceinline__ int64_t load_cu(const void* cu, int is64, int i) {
  return is64 ? static_cast<const int64_t*>(cu)[i] : int64_t(static_cast<const int32_t*>(cu)[i]);
}

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_inclusive_scan(float x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x;
}

// ---------------------------------------------------------------------------
// T~ = (I + N)^-1 for strictly lower N (64x64 fp32 in LDS), by 2x2 block
// recursion: 16x16 diagonal blocks by forward substitution, then
// inv([A 0; C B]) = [A^-1 0; -B^-1 C A^-1  B^-1] at sizes 32 and 64.
// The lower-triangular result is built in X; the strictly-upper blocks of N
// (never written by the caller) hold the C A^-1 intermediates, and the
// upper 16x16 blocks of X that the products read are zeroed first.
// Called by all 256 threads; ends with a barrier.
// ---------------------------------------------------------------------------
__device__ void solve_unit_lower(PrefillSmem& sm, int tid) {
  float* N = sm.N;
  float* X = sm.X;
  if (tid < 64) {                                   // diagonal 16x16 blocks
    const int I = tid >> 4, j = tid & 15, base = 16 * I;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (i == j) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      const float* nrow = N + (base + i) * FSTR + base;
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc += nrow[m] * x[m];
      if (i > j) x[i] = -acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) X[(base + i) * FSTR + base + j] = x[i];
  } else {                                          // zero X[b..b+16][b+16..b+32], b = 0, 32
    for (int e = tid - 64; e < 512; e += NTHREADS - 64) {
      const int b = 32 * (e >> 8), r = (e >> 4) & 15, c = e & 15;
      X[(b + r) * FSTR + b + 16 + c] = 0.f;
    }
  }
  __syncthreads();
  {                                                 // E = N[b+16.., b..] D_lo  -> N[b+r][b+16+c]
    const int p = tid >> 7, r = (tid >> 3) & 15, c0 = (tid & 7) * 2, b = 32 * p;
    float e0 = 0.f, e1 = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float n = N[(b + 16 + r) * FSTR + b + m];
      e0 += n * X[(b + m) * FSTR + b + c0];
      e1 += n * X[(b + m) * FSTR + b + c0 + 1];
    }
    N[(b + r) * FSTR + b + 16 + c0] = e0;
    N[(b + r) * FSTR + b + 16 + c0 + 1] = e1;
  }
  __syncthreads();
  {                                                 // X[b+16+r][b+c] = -D_hi E
    const int p = tid >> 7, r = (tid >> 3) & 15, c0 = (tid & 7) * 2, b = 32 * p;
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float d = X[(b + 16 + r) * FSTR + b + 16 + m];
      x0 += d * N[(b + m) * FSTR + b + 16 + c0];
      x1 += d * N[(b + m) * FSTR + b + 16 + c0 + 1];
    }
    X[(b + 16 + r) * FSTR + b + c0] = -x0;
    X[(b + 16 + r) * FSTR + b + c0 + 1] = -x1;
  }
  __syncthreads();
  {                                                 // F = N[32.., 0..32] X[0..32, 0..32] -> N[r][32+c]
    const int r = tid >> 3, c0 = (tid & 7) * 4;
    float f[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int m = 0; m < 32; ++m) {
      const float n = N[(32 + r) * FSTR + m];
      const float4 xr = *reinterpret_cast<const float4*>(X + m * FSTR + c0);
      f[0] += n * xr.x; f[1] += n * xr.y; f[2] += n * xr.z; f[3] += n * xr.w;
    }
    *reinterpret_cast<float4*>(N + r * FSTR + 32 + c0) = make_float4(f[0], f[1], f[2], f[3]);
  }
  __syncthreads();
  {                                                 // X[32+r][c] = -X[32.., 32..] F
    const int r = tid >> 3, c0 = (tid & 7) * 4;
    float x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int m = 0; m < 32; ++m) {
      const float d = X[(32 + r) * FSTR + 32 + m];
      const float4 fr = *reinterpret_cast<const float4*>(N + m * FSTR + 32 + c0);
      x[0] += d * fr.x; x[1] += d * fr.y; x[2] += d * fr.z; x[3] += d * fr.w;
    }
    *reinterpret_cast<float4*>(X + (32 + r) * FSTR + c0) = make_float4(-x[0], -x[1], -x[2], -x[3]);
  }
  __syncthreads();
}

__global__ __launch_bounds__(NTHREADS) void gdn_prefill_kernel(PrefillArgs p) {
  __shared__ PrefillSmem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;       // k-group of the lane in MFMA layouts
  const int n16 = lane & 15;     // row/column of the lane in MFMA layouts

  const int seq = blockIdx.x / p.Hv;
  const int h = blockIdx.x % p.Hv;
  const int hq = h / (p.Hv / p.Hq);
  const int hk = h / (p.Hv / p.Hk);

  int64_t s0 = load_cu(p.cu_seqlens, p.cu_is_64, seq);
  int64_t s1 = load_cu(p.cu_seqlens, p.cu_is_64, seq + 1);
  s0 = s0 < 0 ? 0 : (s0 > p.T ? p.T : s0);
  s1 = s1 < s0 ? s0 : (s1 > p.T ? p.T : s1);

  // State slab of this wave: rows v = 32*wave + 16*vt + n16, cols k = 16*kt + 4g + i.
  const int64_t state_head = (int64_t(seq) * p.Hv + h) * D * D;
  f32x4 S[2][8];
#pragma unroll
  for (int vt = 0; vt < 2; ++vt) {
    const int v = 32 * wave + 16 * vt + n16;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      if (p.state) {
        const float4 x = *reinterpret_cast<const float4*>(p.state + state_head + int64_t(v) * D + 16 * kt + 4 * g);
        S[vt][kt] = f32x4{x.x, x.y, x.z, x.w};
      } else {
        S[vt][kt] = zero4();
      }
    }
  }

  if (s1 > s0) {
    // P's strictly-upper 16x16 blocks are read by the P v_new product but never
    // written per chunk: zero the whole tile once (the first barrier of the chunk
    // loop orders this before any read).
    for (int e = tid; e < C * TSTR / 8; e += NTHREADS)
      reinterpret_cast<uint4*>(sm.P)[e] = uint4{0u, 0u, 0u, 0u};
    const float A_log = p.A_log[h];
    const float dt_bias = p.dt_bias[h];
    const int64_t q_stride = int64_t(p.Hq) * D;   // token stride of q
    const int64_t k_stride = int64_t(p.Hk) * D;   // token stride of k
    const int64_t v_stride = int64_t(p.Hv) * D;   // token stride of v / out

    for (int64_t cs = s0; cs < s1; cs += C) {
      const int clen = int(s1 - cs < C ? s1 - cs : C);
      __syncthreads();  // the previous chunk's LDS reads are done

      // ---- stage K, Q, V and K^T; wave w loads column segment 4*it + w ------
      // of all 64 tokens, so the K^T writes of one instruction fill one row.
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int c = lane, sg = 4 * it + wave;    // token, 8-column segment
        uint4 kv = uint4{0u, 0u, 0u, 0u}, qv = kv, vv = kv;
        if (c < clen) {
          kv = *reinterpret_cast<const uint4*>(p.k + (cs + c) * k_stride + int64_t(hk) * D + 8 * sg);
          qv = *reinterpret_cast<const uint4*>(p.q + (cs + c) * q_stride + int64_t(hq) * D + 8 * sg);
          vv = *reinterpret_cast<const uint4*>(p.v + (cs + c) * v_stride + int64_t(h) * D + 8 * sg);
        }
        const int col0 = (8 * sg) & ~31, r0 = (8 * sg) & 31;
        const int pa = col0 + perm32(r0), pb = col0 + perm32(r0 + 4);
        *reinterpret_cast<uint2*>(sm.K + c * KSTR + pa) = uint2{kv.x, kv.y};
        *reinterpret_cast<uint2*>(sm.K + c * KSTR + pb) = uint2{kv.z, kv.w};
        *reinterpret_cast<uint2*>(sm.Q + c * KSTR + pa) = uint2{qv.x, qv.y};
        *reinterpret_cast<uint2*>(sm.Q + c * KSTR + pb) = uint2{qv.z, qv.w};
        *reinterpret_cast<uint4*>(sm.V + c * KSTR + 8 * sg) = vv;
        const int pc = perm(c);
        const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          sm.Kt[(8 * sg + e) * TSTR + pc] = uint16_t(e & 1 ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
      }
      if (wave == 0) {
        float lg = 0.f, bt = 0.f;
        if (lane < clen) {
          const int64_t idx = (cs + lane) * p.Hv + h;
          lg = log_gate(A_log, bf16_to_f32(p.a[idx]), dt_bias);
          bt = sigmoidf_(bf16_to_f32(p.b[idx]));
        }
        const float gm = wave_inclusive_scan(lg, lane);
        const float glast = readlane_f(gm, clen - 1);
        sm.gam[lane] = gm;
        sm.bet[lane] = bt;
        sm.eg[lane] = expf(gm);
        sm.dd[lane] = expf(glast - gm);
      }
      __syncthreads();

      // ---- N = strictLower(beta Gamma KK^T), P = tril(Gamma QK^T) ------------
      // 20 tiles: 10 lower tiles of KK^T (I >= J) and 10 tiles of K Q^T with
      // row tile J <= column tile I; wave w takes tiles w, w+4, ...
      for (int t = wave; t < 20; t += 4) {
        const int tt = t < 10 ? t : t - 10;
        int I = 0;
        while ((I + 1) * (I + 2) / 2 <= tt) ++I;
        const int J = tt - I * (I + 1) / 2;           // J <= I
        f32x4 acc = zero4();
        if (t < 10) {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            acc = mfma(frag(sm.K, KSTR, 16 * I, ks, lane), frag(sm.K, KSTR, 16 * J, ks, lane), acc);
          // acc[i] = k_r . k_c, r = 16I + 4g + i, c = 16J + n16
          const int c = 16 * J + n16;
          const float gc = sm.gam[c];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * I + 4 * g + i;
            sm.N[r * FSTR + c] = r > c ? sm.bet[r] * exp_le0(sm.gam[r] - gc) * acc[i] : 0.f;
          }
        } else {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            acc = mfma(frag(sm.K, KSTR, 16 * J, ks, lane), frag(sm.Q, KSTR, 16 * I, ks, lane), acc);
          // acc[i] = k_j . q_c, j = 16J + 4g + i, c = 16I + n16  ->  P[c][j]
          const int c = 16 * I + n16;
          const float gc = sm.gam[c];
          float pv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * J + 4 * g + i;
            pv[i] = j <= c ? exp_le0(gc - sm.gam[j]) * acc[i] : 0.f;
          }
          *reinterpret_cast<uint2*>(sm.P + c * TSTR + perm(16 * J + 4 * g)) =
              uint2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
        }
      }
      __syncthreads();

      // ---- T~ = (I + N)^-1, stored as bf16 hi/lo with permuted columns ------
      solve_unit_lower(sm, tid);
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int grp = tid + it * NTHREADS;   // 1024 groups of 4 columns
        const int c = grp >> 4, j0 = (grp & 15) * 4;
        f32x4 x;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = j0 + i;
          x[i] = j < c ? sm.X[c * FSTR + j] : (j == c ? 1.f : 0.f);
        }
        const uint32_t h0 = pack_bf16x2(x[0], x[1]), h1 = pack_bf16x2(x[2], x[3]);
        const int pj = perm(j0);
        *reinterpret_cast<uint2*>(sm.Th + c * TSTR + pj) = uint2{h0, h1};
        *reinterpret_cast<uint2*>(sm.Tl + c * TSTR + pj) = uint2{lo_word(x[0], x[1], h0), lo_word(x[2], x[3], h1)};
      }
      __syncthreads();

      // ---- state-dependent part (registers + read-only LDS) -----------------
      // S as B operand (contraction over k): hi/lo for k-blocks ks = 0..3.
      uint4 Sh[2][4], Sl[2][4];
#pragma unroll
      for (int vt = 0; vt < 2; ++vt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) split_pack(S[vt][2 * ks], S[vt][2 * ks + 1], Sh[vt][ks], Sl[vt][ks]);

      // X = K S^T and Q S^T for this wave's 32 columns v (rows c of 4 tiles).
      f32x4 Xk[4][2], Xq[4][2];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) { Xk[ct][vt] = zero4(); Xq[ct][vt] = zero4(); }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint4 ak = frag(sm.K, KSTR, 16 * ct, ks, lane);
          const uint4 aq = frag(sm.Q, KSTR, 16 * ct, ks, lane);
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) {
            Xk[ct][vt] = mfma(ak, Sh[vt][ks], Xk[ct][vt]);
            Xk[ct][vt] = mfma(ak, Sl[vt][ks], Xk[ct][vt]);
            Xq[ct][vt] = mfma(aq, Sh[vt][ks], Xq[ct][vt]);
            Xq[ct][vt] = mfma(aq, Sl[vt][ks], Xq[ct][vt]);
          }
        }
      }

      // Y = beta (V - e^gamma X); element (c = 16ct + 4g + i, v = 32w + 16vt + n16).
      // The inter term e^gamma_c (Q S^T)[c] is scaled here too.
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = 16 * ct + 4 * g + i;
          const float bc = sm.bet[c], ec = sm.eg[c];
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) {
            const float vval = bf16_to_f32(sm.V[c * KSTR + 32 * wave + 16 * vt + n16]);
            Xk[ct][vt][i] = bc * (vval - ec * Xk[ct][vt][i]);
            Xq[ct][vt][i] *= ec;
          }
        }

      // v_new = T~ Y  (contraction over j = rows of Y: blocks js = 0, 1).
      uint4 Yh[2][2], Yl[2][2];
#pragma unroll
      for (int vt = 0; vt < 2; ++vt)
#pragma unroll
        for (int js = 0; js < 2; ++js) split_pack(Xk[2 * js][vt], Xk[2 * js + 1][vt], Yh[vt][js], Yl[vt][js]);
      f32x4 Vn[4][2];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) Vn[ct][vt] = zero4();
#pragma unroll
        for (int js = 0; js <= (ct >> 1); ++js) {     // T~ is lower triangular
          const uint4 th = frag(sm.Th, TSTR, 16 * ct, js, lane);
          const uint4 tl = frag(sm.Tl, TSTR, 16 * ct, js, lane);
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) {
            Vn[ct][vt] = mfma(th, Yh[vt][js], Vn[ct][vt]);
            Vn[ct][vt] = mfma(th, Yl[vt][js], Vn[ct][vt]);
            Vn[ct][vt] = mfma(tl, Yh[vt][js], Vn[ct][vt]);
          }
        }
      }

      // o = scale (e^gamma Q S^T + P v_new), staged in LDS for coalesced stores.
      uint4 Vb[2][2];
#pragma unroll
      for (int vt = 0; vt < 2; ++vt)
#pragma unroll
        for (int js = 0; js < 2; ++js) Vb[vt][js] = pack_hi(Vn[2 * js][vt], Vn[2 * js + 1][vt]);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
        for (int js = 0; js <= (ct >> 1); ++js) {     // P is lower triangular
          const uint4 pa = frag(sm.P, TSTR, 16 * ct, js, lane);
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) Xq[ct][vt] = mfma(pa, Vb[vt][js], Xq[ct][vt]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int vt = 0; vt < 2; ++vt)
            sm.O[(16 * ct + 4 * g + i) * KSTR + 32 * wave + 16 * vt + n16] = f32_to_bf16(p.scale * Xq[ct][vt][i]);
      }

      // S = e^{gamma_last} S + sum_c K[c]^T (d_c v_new[c]),  d_c = e^{gamma_last - gamma_c}
      const float dlast = sm.eg[clen - 1];
      uint4 Uh[2][2], Ul[2][2];
#pragma unroll
      for (int js = 0; js < 2; ++js) {
        const float4 d0 = *reinterpret_cast<const float4*>(sm.dd + 32 * js + 4 * g);
        const float4 d1 = *reinterpret_cast<const float4*>(sm.dd + 32 * js + 16 + 4 * g);
        const f32x4 e0 = {d0.x, d0.y, d0.z, d0.w}, e1 = {d1.x, d1.y, d1.z, d1.w};
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) split_pack(Vn[2 * js][vt] * e0, Vn[2 * js + 1][vt] * e1, Uh[vt][js], Ul[vt][js]);
      }
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) S[vt][kt] = S[vt][kt] * dlast;
#pragma unroll
        for (int js = 0; js < 2; ++js) {
          const uint4 ak = frag(sm.Kt, TSTR, 16 * kt, js, lane);
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) {
            S[vt][kt] = mfma(ak, Uh[vt][js], S[vt][kt]);
            S[vt][kt] = mfma(ak, Ul[vt][js], S[vt][kt]);
          }
        }
      }

      __syncthreads();  // output tile complete
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int seg = tid + it * NTHREADS;
        const int c = seg >> 4, sg = seg & 15;
        if (c < clen)
          *reinterpret_cast<uint4*>(p.out + (cs + c) * v_stride + int64_t(h) * D + 8 * sg) =
              *reinterpret_cast<const uint4*>(sm.O + c * KSTR + 8 * sg);
      }
    }
  }

  // Final state (for an empty sequence: the initial state, or zeros).
  if (s1 > s0 || p.state != p.new_state) {
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      const int v = 32 * wave + 16 * vt + n16;
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        const f32x4 x = S[vt][kt];
        *reinterpret_cast<float4*>(p.new_state + state_head + int64_t(v) * D + 16 * kt + 4 * g) =
            make_float4(x[0], x[1], x[2], x[3]);
      }
    }
  }
}

}  // namespace

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  const int64_t grid = int64_t(a.N) * a.Hv;
  hipLaunchKernelGGL(gdn_prefill_kernel, dim3(unsigned(grid)), dim3(NTHREADS), 0, stream, a);
  return hipGetLastError();
}

}  // namespace gdn

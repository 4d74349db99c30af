// GDN varlen chunked prefill for gfx950 (chunk C = 64, dk = dv = 128).
//
// One workgroup of 4 wavefronts walks the chunks of one (sequence, v-head)
// chain.  The fp32 state never leaves the register file between chunks: wave w
// owns state rows v in [32w, 32w+32) as MFMA accumulators (16x16 tiles of S^T;
// lane = (k-group g = lane/16, column n = lane%16) holds S[v][k..k+3]).
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
// Work split inside a chunk (all waves in parallel between barriers):
//   A: wave 0 -- the four diagonal 16x16 blocks of N and their inverses (VALU
//      forward substitution); waves 1, 2 -- the off-diagonal blocks of N (bf16
//      hi/lo) and P; wave 3 -- two blocks of P and its X = K S^T.
//   B: wave 3 -- the off-diagonal blocks of T~ by block recursion on MFMA;
//      waves 0-2 -- their X = K S^T; wave 1 also the next chunk's gates.
//   C: every wave -- Y, v_new, the output, the state update; the next chunk's
//      inputs are loaded into registers meanwhile.
//
// Precision: q/k/v are exact bf16 MFMA operands.  Operands that are fp32 values
// (S, Y, N, T~, d*v_new) are split into bf16 hi + lo pairs so that the products
// feeding the state carry ~16 mantissa bits; fp32 accumulation throughout.  The
// output-only products (Q S^T and P v_new) use bf16 hi parts alone.
//
// MFMA operand convention (v_mfma_f32_16x16x32_bf16): lane l supplies row/col
// l%16 and 8 contraction elements chosen by g = l/16.  A and B are paired with
// contraction index kappa(g, s) = 4g + s (s < 4), 16 + 4g + (s - 4) (s >= 4)
// inside each 32-wide block -- exactly what two 16x16 accumulator tiles stacked
// along the contraction dim hold, so accumulators become A or B operands without
// leaving registers.  LDS tiles keep their contraction columns in that order
// (perm32) so an operand row is one 16-byte read; an operand column of a
// row-major tile is two ds_read_b64_tr_b16 (transpose reads within 16 lanes).
#include "gdn_common.hpp"
#include "gdn_launch.hpp"

namespace gdn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int C = 64;        // chunk length
constexpr int D = kHeadDim;  // 128
constexpr int KSTR = 136;    // bf16 row stride of 128-wide tiles (K, Q, V, O)
constexpr int TSTR = 72;     // bf16 row stride of 64-wide tiles (T~, P, N)
constexpr int DSTR = 17;     // fp32 row stride of the diagonal N blocks
constexpr int NTHREADS = 256;
constexpr int kMaxSortedSeqs = 1024;  // longest-first ordering up to this many sequences

struct __align__(16) PrefillSmem {
  uint16_t K[C * KSTR];       // K chunk [c][perm(k)]
  uint16_t Q[C * KSTR];       // Q chunk [c][perm(k)]
  uint16_t V[C * KSTR];       // V chunk [c][v]
  uint16_t O[C * KSTR];       // output tile [c][v]; sequence lengths at kernel start
  uint16_t Th[C * TSTR];      // T~ hi [c][perm(j)] (strictly-upper blocks stay 0)
  uint16_t Tl[C * TSTR];      // T~ lo
  uint16_t P[C * TSTR];       // P (bf16) [c][perm(j)]
  uint16_t Nh[C * TSTR];      // off-diagonal blocks of N, hi [i][perm(j)]
  uint16_t Nl[C * TSTR];      // off-diagonal blocks of N, lo
  float Nd[4 * 16 * DSTR];    // diagonal 16x16 blocks of N (fp32)
  // Per-chunk gate values, double-buffered (chunk parity): the next chunk's are
  // written while the current chunk's are read.
  float gam[2][C];            // gamma_c (inclusive cumsum of the log gates)
  float bet[2][C];            // beta_c
  float eg[2][C];             // e^{gamma_c}
  float dd[2][C];             // e^{gamma_last - gamma_c}
  int seq;                    // sequence handled by this workgroup
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

// Operand row: rows row0 + lane%16, contraction block ks (32 wide), from a tile
// stored with permuted columns.
__device__ __forceinline__ uint4 frag(const uint16_t* tile, int stride, int row0, int ks, int lane) {
  return *reinterpret_cast<const uint4*>(tile + (row0 + (lane & 15)) * stride + 32 * ks + 8 * (lane >> 4));
}

__device__ __forceinline__ uint2 read_tr(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

// Operand column: column col0 + lane%16 of a row-major tile, contraction rows
// k0 + kappa(g, s).  In each 16-lane group, lane j reads 4 contiguous columns of
// row k0 + 4g + j/4 (+16 for the second half); the transpose read hands lane i
// element i of each of those rows.  PERM: the tile's columns are perm-ordered.
template <bool PERM>
__device__ __forceinline__ uint4 frag_tr(const uint16_t* tile, int stride, int k0, int col0, int lane) {
  const int j = lane & 15, g = lane >> 4;
  const int col = col0 + 4 * (j & 3);
  const uint16_t* ptr = tile + (k0 + 4 * g + (j >> 2)) * stride + (PERM ? perm(col) : col);
  const uint2 a = read_tr(ptr);
  const uint2 b = read_tr(ptr + 16 * stride);
  return uint4{a.x, a.y, b.x, b.y};
}

// Four rows k0 + 4g .. +3 of column col0 + lane%16 (the first half of frag_tr).
__device__ __forceinline__ uint2 col4_tr(const uint16_t* tile, int stride, int k0, int col0, int lane) {
  const int j = lane & 15, g = lane >> 4;
  return read_tr(tile + (k0 + 4 * g + (j >> 2)) * stride + col0 + 4 * (j & 3));
}

// B/A operand (bf16 hi parts) from two accumulator tiles stacked along the
// contraction dim.
__device__ __forceinline__ uint4 pack_hi(const f32x4& t0, const f32x4& t1) {
  return uint4{pack_bf16x2(t0[0], t0[1]), pack_bf16x2(t0[2], t0[3]), pack_bf16x2(t1[0], t1[1]),
               pack_bf16x2(t1[2], t1[3])};
}
// bf16 lo parts x - hi(x) (exact in fp32), rounded to bf16, given the hi word.
__device__ __forceinline__ uint32_t lo_word(float a, float b, uint32_t hi) {
  return pack_bf16x2(a - bf16lo_f32(hi), b - bf16hi_f32(hi));
}
__device__ __forceinline__ void split_pack(const f32x4& t0, const f32x4& t1, uint4& hi, uint4& lo) {
  hi = pack_hi(t0, t1);
  lo = uint4{lo_word(t0[0], t0[1], hi.x), lo_word(t0[2], t0[3], hi.y), lo_word(t1[0], t1[1], hi.z),
             lo_word(t1[2], t1[3], hi.w)};
}
__device__ __forceinline__ void split4(const f32x4& t, uint2& hi, uint2& lo) {
  hi = uint2{pack_bf16x2(t[0], t[1]), pack_bf16x2(t[2], t[3])};
  lo = uint2{lo_word(t[0], t[1], hi.x), lo_word(t[2], t[3], hi.y)};
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

// Orders this wave's LDS writes before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// Tiles of N and P from the staged K and Q (16x16 tiles, 4 MFMAs each).
//   kind 0: diagonal block I of N (fp32, into Nd), from tile K_I K_I^T
//   kind 1: off-diagonal block (I, J), I > J, of N (bf16 hi/lo), from tile
//           K_J K_I^T so that a lane holds 4 consecutive columns of one row
//   kind 2: block (I, J), J <= I, of P, from tile K_J Q_I^T
// ---------------------------------------------------------------------------
struct TileJob {
  int kind, I, J;
};

__device__ __forceinline__ void tile_epilogue(PrefillSmem& sm, int buf, const TileJob t, const f32x4& acc, int lane) {
  const int g = lane >> 4, n16 = lane & 15;
  const float* gam = sm.gam[buf];
  const float* bet = sm.bet[buf];
  if (t.kind == 0) {
    // acc[i] = k_r . k_c, r = 16I + 4g + i, c = 16I + n16
    const int c = 16 * t.I + n16;
    const float gc = gam[c];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ri = 4 * g + i, r = 16 * t.I + ri;
      sm.Nd[(t.I * 16 + ri) * DSTR + n16] = ri > n16 ? bet[r] * exp_le0(gam[r] - gc) * acc[i] : 0.f;
    }
  } else if (t.kind == 1) {
    // acc[i] = k_c . k_r, c = 16J + 4g + i, r = 16I + n16  ->  N[r][c]
    const int r = 16 * t.I + n16;
    const float gr = gam[r], br = bet[r];
    f32x4 x;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = br * exp_le0(gr - gam[16 * t.J + 4 * g + i]) * acc[i];
    uint2 hi, lo;
    split4(x, hi, lo);
    const int pos = r * TSTR + perm(16 * t.J + 4 * g);
    *reinterpret_cast<uint2*>(sm.Nh + pos) = hi;
    *reinterpret_cast<uint2*>(sm.Nl + pos) = lo;
  } else {
    // acc[i] = k_j . q_c, j = 16J + 4g + i, c = 16I + n16  ->  P[c][j]
    const int c = 16 * t.I + n16;
    const float gc = gam[c];
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 16 * t.J + 4 * g + i;
      pv[i] = j <= c ? exp_le0(gc - gam[j]) * acc[i] : 0.f;
    }
    *reinterpret_cast<uint2*>(sm.P + c * TSTR + perm(16 * t.J + 4 * g)) =
        uint2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
  }
}

template <int NJ>
__device__ __forceinline__ void run_tiles(PrefillSmem& sm, int buf, const TileJob (&jobs)[NJ], int lane) {
  f32x4 acc[NJ];
#pragma unroll
  for (int t = 0; t < NJ; ++t) acc[t] = zero4();
#pragma unroll 1
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      const TileJob j = jobs[t];
      const int arow = j.kind == 0 ? 16 * j.I : 16 * j.J;
      const uint16_t* btile = j.kind == 2 ? sm.Q : sm.K;
      const int brow = 16 * j.I;
      acc[t] = mfma(frag(sm.K, KSTR, arow, ks, lane), frag(btile, KSTR, brow, ks, lane), acc[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < NJ; ++t) tile_epilogue(sm, buf, jobs[t], acc[t], lane);
}

// ---------------------------------------------------------------------------
// Diagonal blocks of T~: D_I = (I + N_II)^-1 by forward substitution; lane
// 16I + j owns column j of block I.  Written to Th/Tl (including the zero
// upper part and the unit diagonal of each block).  One wavefront.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void solve_diagonal(PrefillSmem& sm, int lane) {
  const int I = lane >> 4, j = lane & 15;
  const float* nb = sm.Nd + I * 16 * DSTR;
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = (i == j) ? 1.f : 0.f;
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    float acc0 = 0.f, acc1 = 0.f;   // two partial sums halve the dependent FMA chain
#pragma unroll
    for (int m = 0; m < i; m += 2) {
      acc0 += nb[i * DSTR + m] * x[m];
      if (m + 1 < i) acc1 += nb[i * DSTR + m + 1] * x[m + 1];
    }
    if (i > j) x[i] = -(acc0 + acc1);
    if (i & 1) __builtin_amdgcn_sched_barrier(0);  // bound hoisted LDS reads to ~two rows
  }
  const int col = perm(16 * I + j);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint16_t hi = f32_to_bf16(x[i]);
    sm.Th[(16 * I + i) * TSTR + col] = hi;
    sm.Tl[(16 * I + i) * TSTR + col] = f32_to_bf16(x[i] - bf16_to_f32(hi));
  }
}

// ---------------------------------------------------------------------------
// Off-diagonal blocks of T~ (one wavefront, MFMA with hi/lo operands):
//   X_IJ = -D_I G_IJ,  G_IJ = sum_{K=J}^{I-1} N_IK X_KJ  (X_JJ = D_J)
// in three dependency levels: (1,0) (2,1) (3,2); (2,0) (3,1); (3,0).
// A operands: rows of N (Nh/Nl) and of T~ (Th/Tl); B operands: the stacked
// blocks X_KJ read as columns of Th/Tl, or G from registers.  Halves of a 32-wide
// contraction block that fall outside K in [J, I-1] are zeroed in B.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint4 keep_halves(uint4 b, bool lo_half, bool hi_half) {
  if (!lo_half) { b.x = 0u; b.y = 0u; }
  if (!hi_half) { b.z = 0u; b.w = 0u; }
  return b;
}

__device__ __forceinline__ f32x4 g_pass(const PrefillSmem& sm, f32x4 G, int I, int J, int q, bool klo, bool khi,
                                        int lane) {
  const uint4 ah = frag(sm.Nh, TSTR, 16 * I, q, lane), al = frag(sm.Nl, TSTR, 16 * I, q, lane);
  const uint4 bh = keep_halves(frag_tr<true>(sm.Th, TSTR, 32 * q, 16 * J, lane), klo, khi);
  const uint4 bl = keep_halves(frag_tr<true>(sm.Tl, TSTR, 32 * q, 16 * J, lane), klo, khi);
  G = mfma(ah, bh, G);
  G = mfma(ah, bl, G);
  G = mfma(al, bh, G);
  return G;
}

// X_IJ = -D_I G, written to Th/Tl.
__device__ __forceinline__ void finish_block(PrefillSmem& sm, const f32x4& G, int I, int J, int lane) {
  uint2 gh, gl;
  split4(G, gh, gl);
  const bool odd = I & 1;
  const uint4 bh = odd ? uint4{0u, 0u, gh.x, gh.y} : uint4{gh.x, gh.y, 0u, 0u};
  const uint4 bl = odd ? uint4{0u, 0u, gl.x, gl.y} : uint4{gl.x, gl.y, 0u, 0u};
  const uint4 ah = frag(sm.Th, TSTR, 16 * I, I >> 1, lane), al = frag(sm.Tl, TSTR, 16 * I, I >> 1, lane);
  f32x4 X = zero4();
  X = mfma(ah, bh, X);
  X = mfma(ah, bl, X);
  X = mfma(al, bh, X);
  const int g = lane >> 4, col = perm(16 * J + (lane & 15));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x = -X[i];
    const uint16_t hi = f32_to_bf16(x);
    sm.Th[(16 * I + 4 * g + i) * TSTR + col] = hi;
    sm.Tl[(16 * I + 4 * g + i) * TSTR + col] = f32_to_bf16(x - bf16_to_f32(hi));
  }
}

__device__ __forceinline__ void solve_offdiagonal(PrefillSmem& sm, int lane) {
  // level 1
  const f32x4 g10 = g_pass(sm, zero4(), 1, 0, 0, true, false, lane);
  const f32x4 g21 = g_pass(sm, zero4(), 2, 1, 0, false, true, lane);
  const f32x4 g32 = g_pass(sm, zero4(), 3, 2, 1, true, false, lane);
  finish_block(sm, g10, 1, 0, lane);
  finish_block(sm, g21, 2, 1, lane);
  finish_block(sm, g32, 3, 2, lane);
  wave_lds_sync();
  // level 2
  const f32x4 g20 = g_pass(sm, zero4(), 2, 0, 0, true, true, lane);
  f32x4 g31 = g_pass(sm, zero4(), 3, 1, 0, false, true, lane);
  g31 = g_pass(sm, g31, 3, 1, 1, true, false, lane);
  finish_block(sm, g20, 2, 0, lane);
  finish_block(sm, g31, 3, 1, lane);
  wave_lds_sync();
  // level 3
  f32x4 g30 = g_pass(sm, zero4(), 3, 0, 0, true, true, lane);
  g30 = g_pass(sm, g30, 3, 0, 1, true, false, lane);
  finish_block(sm, g30, 3, 0, lane);
}

// X = K S^T (rows c, cols v: Xk[ct][vt]) for this wave's 32 state rows; S
// enters as hi/lo B operands.
__device__ __forceinline__ void retrieve(const PrefillSmem& sm, const f32x4 (&S)[2][8], f32x4 (&Xk)[4][2], int lane) {
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) Xk[ct][vt] = zero4();
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 Sh[2], Sl[2];
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) split_pack(S[vt][2 * ks], S[vt][2 * ks + 1], Sh[vt], Sl[vt]);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const uint4 ak = frag(sm.K, KSTR, 16 * ct, ks, lane);
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        Xk[ct][vt] = mfma(ak, Sh[vt], Xk[ct][vt]);
        Xk[ct][vt] = mfma(ak, Sl[vt], Xk[ct][vt]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // bound the number of operand loads in flight
  }
}

// (Q S^T)^T (rows v, cols c: Xq[vt][ct]) for this wave's 32 state rows; S enters
// as the bf16 hi A operand (output-only product).
__device__ __forceinline__ void inter_term(const PrefillSmem& sm, const f32x4 (&S)[2][8], f32x4 (&Xq)[2][4],
                                           int lane) {
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) Xq[vt][ct] = zero4();
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 Sh[2];
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) Sh[vt] = pack_hi(S[vt][2 * ks], S[vt][2 * ks + 1]);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const uint4 bq = frag(sm.Q, KSTR, 16 * ct, ks, lane);
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) Xq[vt][ct] = mfma(Sh[vt], bq, Xq[vt][ct]);
    }
  }
}

struct Prefetch {
  uint4 k[4], q[4], v[4];
};

// This thread's K/Q/V segments of a chunk: segment tid + 256*it is token
// seg/16, columns 8*(seg%16) .. +7, so 16 consecutive threads read one
// contiguous 256-byte row.
__device__ __forceinline__ void prefetch_chunk(const PrefillArgs& p, int64_t cs, int clen, int h, int hq, int hk,
                                               int tid, Prefetch& f) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int seg = tid + it * NTHREADS, c = seg >> 4, sg = seg & 15;
    f.k[it] = f.q[it] = f.v[it] = uint4{0u, 0u, 0u, 0u};
    if (c < clen) {
      f.k[it] = *reinterpret_cast<const uint4*>(p.k + ((cs + c) * p.Hk + hk) * D + 8 * sg);
      f.q[it] = *reinterpret_cast<const uint4*>(p.q + ((cs + c) * p.Hq + hq) * D + 8 * sg);
      f.v[it] = *reinterpret_cast<const uint4*>(p.v + ((cs + c) * p.Hv + h) * D + 8 * sg);
    }
  }
}

// Per-token gate values of a chunk, one token per lane of a wavefront, into
// gate buffer `buf`.
__device__ __forceinline__ void chunk_gates(PrefillSmem& sm, int buf, float a, float b, float A_log, float dt_bias,
                                            int clen, int lane) {
  const float lg = lane < clen ? log_gate(A_log, a, dt_bias) : 0.f;
  const float bt = lane < clen ? sigmoidf_(b) : 0.f;
  const float gm = wave_inclusive_scan(lg, lane);
  const float glast = readlane_f(gm, clen - 1);
  sm.gam[buf][lane] = gm;
  sm.bet[buf][lane] = bt;
  sm.eg[buf][lane] = expf(gm);
  sm.dd[buf][lane] = expf(glast - gm);
}

__device__ __forceinline__ void load_ab(const PrefillArgs& p, int64_t cs, int clen, int h, int lane, float& a,
                                        float& b) {
  a = b = 0.f;
  if (lane < clen) {
    const int64_t idx = (cs + lane) * p.Hv + h;
    a = bf16_to_f32(p.a[idx]);
    b = bf16_to_f32(p.b[idx]);
  }
}

// Workgroup barrier ordering LDS only: waits for this wave's LDS operations,
// not for its outstanding global loads/stores (no global memory is shared
// between the waves of a workgroup here).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The sequence of rank `rank` in descending length order (ties: lower index
// first), so the longest chains start first; natural order for large batches.
__device__ int pick_sequence(PrefillSmem& sm, const PrefillArgs& p, int rank, int tid) {
  if (p.N <= 1 || p.N > kMaxSortedSeqs) return rank;
  int* len = reinterpret_cast<int*>(sm.O);
  for (int i = tid; i < p.N; i += NTHREADS) {
    int64_t a = load_cu(p.cu_seqlens, p.cu_is_64, i), b = load_cu(p.cu_seqlens, p.cu_is_64, i + 1);
    a = a < 0 ? 0 : (a > p.T ? p.T : a);
    b = b < a ? a : (b > p.T ? p.T : b);
    len[i] = int(b - a);
  }
  __syncthreads();
  for (int i = tid; i < p.N; i += NTHREADS) {
    const int li = len[i];
    int r = 0;
    for (int j = 0; j < p.N; ++j) {
      const int lj = len[j];
      r += (lj > li) | ((lj == li) & (j < i));
    }
    if (r == rank) sm.seq = i;
  }
  __syncthreads();
  return sm.seq;
}

__global__ __launch_bounds__(NTHREADS) void gdn_prefill_kernel(PrefillArgs p) {
  __shared__ PrefillSmem sm;

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int h = blockIdx.x % p.Hv;
  const int seq = pick_sequence(sm, p, blockIdx.x / p.Hv, tid);
  const int hq = h / (p.Hv / p.Hq);
  const int hk = h / (p.Hv / p.Hk);

  int64_t s0 = load_cu(p.cu_seqlens, p.cu_is_64, seq);
  int64_t s1 = load_cu(p.cu_seqlens, p.cu_is_64, seq + 1);
  s0 = s0 < 0 ? 0 : (s0 > p.T ? p.T : s0);
  s1 = s1 < s0 ? s0 : (s1 > p.T ? p.T : s1);

  // State slab of this wave: rows v = 32*wave + 16*vt + n16, cols k = 16*kt + 4g + i.
  const int64_t state_head = (int64_t(seq) * p.Hv + h) * D * D;
  f32x4 S[2][8];
  {
  const int g = lane0 >> 4, n16 = lane0 & 15;
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
  }

  if (s1 > s0) {
    // Blocks of T~, N and P that are never written per chunk are read as zeros
    // (strictly-upper blocks, the diagonal blocks of Nh/Nl): clear them once.
    for (int e = tid; e < C * TSTR / 8; e += NTHREADS) {
      reinterpret_cast<uint4*>(sm.P)[e] = uint4{0u, 0u, 0u, 0u};
      reinterpret_cast<uint4*>(sm.Th)[e] = uint4{0u, 0u, 0u, 0u};
      reinterpret_cast<uint4*>(sm.Tl)[e] = uint4{0u, 0u, 0u, 0u};
      reinterpret_cast<uint4*>(sm.Nh)[e] = uint4{0u, 0u, 0u, 0u};
      reinterpret_cast<uint4*>(sm.Nl)[e] = uint4{0u, 0u, 0u, 0u};
    }
    const float A_log = p.A_log[h];
    const float dt_bias = p.dt_bias[h];
    const int64_t out_stride = int64_t(p.Hv) * D;

    Prefetch f;
    {
      const int clen0 = int(s1 - s0 < C ? s1 - s0 : C);
      prefetch_chunk(p, s0, clen0, h, hq, hk, tid, f);
      if (wave == 1) {
        float a, b;
        load_ab(p, s0, clen0, h, lane0, a, b);
        chunk_gates(sm, 0, a, b, A_log, dt_bias, clen0, lane0);
      }
    }
    int buf = 0;   // gate buffer of the current chunk

    for (int64_t cs = s0; cs < s1; cs += C) {
      const int clen = int(s1 - cs < C ? s1 - cs : C);
      // The lane index is re-materialised opaquely each chunk so that the many
      // lane-dependent LDS addresses below are recomputed in the loop instead of
      // being hoisted out of it (and spilled).
      int lane = lane0;
      asm volatile("" : "+v"(lane));
      const int g = lane >> 4, n16 = lane & 15;
      lds_barrier();  // the previous chunk's LDS reads are done

      // ---- stage K, Q, V from the prefetched registers; gates ---------------
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int seg = tid + it * NTHREADS, c = seg >> 4, sg = seg & 15;
        const int col0 = (8 * sg) & ~31, r0 = (8 * sg) & 31;
        const int pa = col0 + perm32(r0), pb = col0 + perm32(r0 + 4);
        *reinterpret_cast<uint2*>(sm.K + c * KSTR + pa) = uint2{f.k[it].x, f.k[it].y};
        *reinterpret_cast<uint2*>(sm.K + c * KSTR + pb) = uint2{f.k[it].z, f.k[it].w};
        *reinterpret_cast<uint2*>(sm.Q + c * KSTR + pa) = uint2{f.q[it].x, f.q[it].y};
        *reinterpret_cast<uint2*>(sm.Q + c * KSTR + pb) = uint2{f.q[it].z, f.q[it].w};
        *reinterpret_cast<uint4*>(sm.V + c * KSTR + 8 * sg) = f.v[it];
      }
      lds_barrier();
      const float* gam = sm.gam[buf];
      const float* bet = sm.bet[buf];
      const float* egv = sm.eg[buf];
      const float* ddv = sm.dd[buf];

      // Next chunk's gate inputs (wave 1): loaded now, turned into gates in phase B.
      const int64_t nc = cs + C;
      const int nclen = int(s1 - nc < C ? s1 - nc : C);
      float na = 0.f, nb = 0.f;
      if (wave == 1 && nc < s1) load_ab(p, nc, nclen, h, lane, na, nb);

      f32x4 Xk[4][2];
      // ---- phase A -------------------------------------------------------------
      if (wave == 0) {
        const TileJob jobs[4] = {{0, 0, 0}, {0, 1, 1}, {0, 2, 2}, {0, 3, 3}};
        run_tiles(sm, buf, jobs, lane);
        wave_lds_sync();
        solve_diagonal(sm, lane);
      } else if (wave == 1) {
        const TileJob jobs[8] = {{1, 1, 0}, {1, 2, 0}, {1, 3, 0}, {1, 2, 1},
                                 {1, 3, 1}, {1, 3, 2}, {2, 0, 0}, {2, 1, 1}};
        run_tiles(sm, buf, jobs, lane);
      } else if (wave == 2) {
        const TileJob jobs[6] = {{2, 1, 0}, {2, 2, 0}, {2, 2, 1}, {2, 2, 2}, {2, 3, 0}, {2, 3, 1}};
        run_tiles(sm, buf, jobs, lane);
      } else {
        const TileJob jobs[2] = {{2, 3, 2}, {2, 3, 3}};
        run_tiles(sm, buf, jobs, lane);
        retrieve(sm, S, Xk, lane);
      }
      lds_barrier();

      // ---- phase B -------------------------------------------------------------
      if (wave == 3) {
        solve_offdiagonal(sm, lane);
      } else {
        retrieve(sm, S, Xk, lane);
        // Next chunk's gates, into the other gate buffer.
        if (wave == 1 && nc < s1) chunk_gates(sm, buf ^ 1, na, nb, A_log, dt_bias, nclen, lane);
      }
      lds_barrier();

      // ---- phase C: Y, v_new, output, state update -------------------------------
      // Y = beta (V - e^gamma X); element (c = 16ct + 4g + i, v = 32w + 16vt + n16).
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const float4 bc = *reinterpret_cast<const float4*>(bet + 16 * ct + 4 * g);
        const float4 ec = *reinterpret_cast<const float4*>(egv + 16 * ct + 4 * g);
        const float b4[4] = {bc.x, bc.y, bc.z, bc.w}, e4[4] = {ec.x, ec.y, ec.z, ec.w};
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) {
          const uint2 vv = col4_tr(sm.V, KSTR, 16 * ct, 32 * wave + 16 * vt, lane);
          const float vf[4] = {bf16lo_f32(vv.x), bf16hi_f32(vv.x), bf16lo_f32(vv.y), bf16hi_f32(vv.y)};
#pragma unroll
          for (int i = 0; i < 4; ++i) Xk[ct][vt][i] = b4[i] * (vf[i] - e4[i] * Xk[ct][vt][i]);
        }
      }

      // v_new = T~ Y (contraction over the rows of Y: blocks js; T~ is lower triangular).
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
        for (int js = 0; js <= (ct >> 1); ++js) {
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

      // o^T = e^gamma (S Q^T) + v_new^T P^T (rows v, cols c); P is lower triangular.
      f32x4 Xq[2][4];
      inter_term(sm, S, Xq, lane);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const float ecn = egv[16 * ct + n16];   // e^gamma of column c = 16ct + n16
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) Xq[vt][ct] = Xq[vt][ct] * ecn;
      }
#pragma unroll
      for (int js = 0; js < 2; ++js) {
        uint4 vb[2];
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) vb[vt] = pack_hi(Vn[2 * js][vt], Vn[2 * js + 1][vt]);
#pragma unroll
        for (int ct = 2 * js; ct < 4; ++ct) {
          const uint4 pb = frag(sm.P, TSTR, 16 * ct, js, lane);
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) Xq[vt][ct] = mfma(vb[vt], pb, Xq[vt][ct]);
        }
      }
      // Lane holds o[c = 16ct + n16][v = 32w + 16vt + 4g .. +3]: one 8-byte LDS write each.
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int c = 16 * ct + n16;
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) {
          const f32x4 o = Xq[vt][ct] * p.scale;
          *reinterpret_cast<uint2*>(sm.O + c * KSTR + 32 * wave + 16 * vt + 4 * g) =
              uint2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        }
      }

      // S = e^{gamma_last} S + sum_c K[c]^T (d_c v_new[c]),  d_c = e^{gamma_last - gamma_c}
      const float dlast = egv[clen - 1];
      uint4 Uh[2][2], Ul[2][2];
#pragma unroll
      for (int js = 0; js < 2; ++js) {
        const float4 d0 = *reinterpret_cast<const float4*>(ddv + 32 * js + 4 * g);
        const float4 d1 = *reinterpret_cast<const float4*>(ddv + 32 * js + 16 + 4 * g);
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
          const uint4 ak = frag_tr<true>(sm.K, KSTR, 32 * js, 16 * kt, lane);
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) {
            S[vt][kt] = mfma(ak, Uh[vt][js], S[vt][kt]);
            S[vt][kt] = mfma(ak, Ul[vt][js], S[vt][kt]);
          }
        }
      }

      lds_barrier();  // output tile complete
      // Next chunk's K/Q/V, in flight during the output store and the barrier.
      if (nc < s1) prefetch_chunk(p, nc, nclen, h, hq, hk, tid, f);
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int seg = tid + it * NTHREADS;
        const int c = seg >> 4, sg = seg & 15;
        if (c < clen)
          *reinterpret_cast<uint4*>(p.out + (cs + c) * out_stride + int64_t(h) * D + 8 * sg) =
              *reinterpret_cast<const uint4*>(sm.O + c * KSTR + 8 * sg);
      }
      buf ^= 1;
    }
  }

  // Final state (for an empty sequence: the initial state, or zeros).
  if (s1 > s0 || p.state != p.new_state) {
    const int g = lane0 >> 4, n16 = lane0 & 15;
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

// GDN varlen chunked prefill for gfx950 (chunk C = 64, dk = dv = 128).
//
// A workgroup walks the chunks of one (sequence, v-head) chain, or of one slice
// of its state rows, as a two-stage pipeline:
//   * NP producer waves (NCW .. NCW+NP-1; four, or seven beside one consumer and six
//     beside two, which fill the workgroup's eight waves)
//     prepare chunk t: stage K and Q in LDS, form the gates, the masked/decayed
//     products N = strictLower(beta Gamma KK^T) and P = tril(Gamma QK^T), and
//     T~ = (I + N)^-1;
//   * the consumer waves (0 .. NCW-1) meanwhile advance the state through chunk t-1.
// Every LDS buffer a consumer reads (K, Q, T~, P, gates) is double-buffered by
// chunk parity (V is single-buffered and rewritten only after it was read).
// The roles hand chunks over through LDS counters, so each runs its own chain
// and neither waits for the other's sub-steps.  The fp32 state never leaves the
// register file: consumer wave w owns state rows v in [R0 + VW w, R0 + VW w + VW)
// as MFMA accumulators (16x16 tiles of S^T; lane = (k-group g = lane/16,
// column n = lane%16) holds S[v][k..k+3]).
//
// Launch variants (struct Variant): NCW consumer waves of VT 16-row tiles each
// cover ROWS = 16 NCW VT state rows, so F = 128 / ROWS workgroups share a chain,
// each owning rows [R0, R0 + ROWS).  They all prepare the same chunk data (the
// producer work does not depend on the state) and each stages only its slice of
// V.  Batches with many chains use F = 1 (four consumer waves of 32 rows); few
// chains are split so that every CU gets a workgroup (with F = 8 and F = 4 one or
// two 16-row consumers beside seven or six pipelined producers, since the chunk
// preparation, repeated in every slice, sets the pace).
// When the caller provides
// a workspace, batches split 4 or 8 ways run in two kernels instead: a prep kernel
// prepares every chunk once (all chunks in parallel), and the state pass's loader
// waves copy its T~/P tiles where the producers would have computed them.
//
// Per chunk (positions >= clen are zero-padded: K = Q = V = 0, beta = 0 and
// log-gate 0, as kernel_prefill.cu:102-114, 125-132 pads them):
//   gamma = inclusive cumsum of the log gates, beta = sigmoid(b)   (a1, :101-122;
//           summed in fp64 and kept as an fp32 pair, in log2 units)
//   N[i][j] = beta_i e^{gamma_i - gamma_j} k_i.k_j   (i > j)       (:134-146, sign folded)
//   P[i][j] = e^{gamma_i - gamma_j} q_i.k_j          (j <= i)       (:165-185; stored times scale)
//   T~ = (I + N)^-1                                   (:148-163)
//   X  = K S^T                                        (retrieval from the chunk-start state)
//   Y  = beta (V - e^gamma X)
//   v_new = T~ Y          (= T~(beta V) - T~(beta e^gamma K) S^T = U - W S^T, :187-195, 236-271)
//   o  = scale (e^gamma Q S^T + P v_new)              (:216-234, 273-283)
//   S  = e^{gamma_last} S + (d v_new)^T K,  d_c = e^{gamma_last - gamma_c}   (:197-202, 286-293)
//
// T~ is built in three steps: each producer wave forms one diagonal 16x16 tile of
// N; one wave inverts the four diagonal blocks D_I = (I + N_II)^-1 by forward
// substitution (16 lanes per block, one lane per column); two waves then form the
// off-diagonal blocks as a 2x2 block inverse over the 32x32 halves on 16x16x16
// MFMAs (offdiag_right / offdiag_left).
//
// Precision: q/k/v are exact bf16 MFMA operands.  Operands that are fp32 values
// (S, Y, N, T~, d*v_new) are split into bf16 hi + lo pairs so that the products
// feeding the state carry ~16 mantissa bits; fp32 accumulation throughout.  The
// output-only products (Q S^T and P v_new) use bf16 hi parts alone.  The residual
// x - hi(x) of a split is formed exactly on the matrix pipe (residual4).
//
// MFMA operand convention (v_mfma_f32_16x16x32_bf16): lane l supplies row/col
// l%16 and 8 contraction elements chosen by g = l/16.  A and B are paired with
// contraction index kappa(g, s) = 4g + s (s < 4), 16 + 4g + (s - 4) (s >= 4)
// inside each 32-wide block -- exactly what two 16x16 accumulator tiles stacked
// along the contraction dim hold, so accumulators become A or B operands without
// leaving registers.  LDS tiles keep their contraction columns in that order
// (perm32) so an operand row is one 16-byte read; an operand column of a
// row-major tile is two ds_read_b64_tr_b16 (transpose reads within 16 lanes).
#include <hip/hip_ext.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_launch.hpp"

namespace gdn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int C = 64;        // chunk length
constexpr int D = kHeadDim;  // 128
constexpr int KSTR = 128;    // bf16 row stride of the K and Q tiles (16-byte slots XOR-swizzled by row)
constexpr int VSTR = 144;    // bf16 row stride of the V tile (rows 32 bytes apart modulo 128)
constexpr int TSTR = 72;     // bf16 row stride of 64-wide tiles (T~, P, N)
constexpr int NDB = 16 * 16 + 4;  // floats per diagonal N block (column-major; padded by 16 bytes)
constexpr int NROWS = C - 16;  // rows of N kept for the off-diagonal solve

template <int NCW_, int VT_, bool HOOKS_ = false, bool LOAD_ = false, int NP_ = 4, bool PERSIST_ = false,
          bool TSPLIT_ = false, bool DEEP_ = false>
struct Variant {
  static constexpr bool kHooks = HOOKS_;         // testing hooks of PrefillArgs compiled in
  static constexpr bool kLoad = LOAD_;           // waves NCW.. load prepared T~/P (two-kernel path)
  static constexpr bool kCopy = false;           // producers copy their tiles out (prep kernel only)
  static constexpr int NCW = NCW_;               // consumer waves
  static constexpr int NP = NP_;                 // producer (or loader) waves: 4; or 7 (6) beside one (two) consumers
  static constexpr int VT = VT_;                 // 16-row state tiles per consumer wave
  static constexpr int VW = 16 * VT;             // state rows per consumer wave
  // Token-split state pass (consumer_loop_tsplit): the consumer waves hold the same
  // 16 state rows and share each chunk's tokens.
  static constexpr bool kTokenSplit = TSPLIT_;
  static constexpr int ROWS = TSPLIT_ ? VW : NCW * VW;  // state rows per workgroup
  static constexpr int F = 128 / ROWS;           // workgroups per chain
  static constexpr int NTHREADS = 64 * (NCW + NP);
  static constexpr int VSEG = 8 * ROWS;          // 16-byte segments of the V slice of a chunk
  // Seven producers beside one consumer, or six beside two, run pipelined one chunk
  // deep (producer_loop_split) with NP - 3 stager waves, and hand a chunk to the
  // consumers in two steps (K, Q, the gates and V; then T~ and P).
  static constexpr bool kPipelined = NP_ >= 6;
  static constexpr int kStagers = NP_ - 3;
  static_assert(F * ROWS == 128 && NCW + NP <= 8, "unsupported launch variant");
  static_assert(NP == 4 || (!LOAD_ && NCW + NP == 8 && NCW <= 2), "pipelined producers fill the workgroup");
  // One workgroup per CU runs a list of whole chains back to back
  // (gdn_prefill_persistent_kernel); the four-producer F = 1 layout only.
  static constexpr bool kPersist = PERSIST_;
  static_assert(!PERSIST_ || (NCW_ == 4 && VT_ == 2 && NP_ == 4 && !LOAD_), "persistent: F = 1 only");
  static_assert(!TSPLIT_ || (NCW_ == 4 && VT_ == 1 && NP_ == 4 && LOAD_ && !PERSIST_), "token split: state pass, F = 8");
  // State pass over images that the caches do not hold (long batches): the loaders
  // load each chunk's images two chunks ahead instead of one.
  static constexpr bool kDeepImages = DEEP_;
  static_assert(!DEEP_ || LOAD_, "image prefetch depth: state pass only");
};

// Production launch variants by split factor F (workgroups per chain).  With F = 8
// (F = 4) a chain's slice has one (two) 16-row consumer waves and the chunk
// preparation, repeated in every slice, sets the pace: seven (six) pipelined
// producer waves share it.
template <bool HOOKS>
using SplitVariant1 = Variant<4, 2, HOOKS>;
template <bool HOOKS>
using SplitVariant2 = Variant<4, 1, HOOKS>;
template <bool HOOKS>
using SplitVariant4 = Variant<2, 1, HOOKS, false, 6>;
template <bool HOOKS>
using SplitVariant8 = Variant<1, 1, HOOKS, false, 7>;
// F = 1 as one workgroup per CU running lists of chains (batches of many chains).
template <bool HOOKS>
using PersistVariant = Variant<4, 2, HOOKS, false, 4, true>;

// The prep kernel of the two-kernel path: the four producer waves alone (no
// consumers, no V staging); they copy each chunk's tiles out themselves (kCopy).
struct PrepVariant {
  static constexpr bool kHooks = false, kCopy = true, kPipelined = false, kPersist = false;
  static constexpr int NCW = 0, NP = 4, ROWS = 128, F = 1;
  static constexpr int NTHREADS = 64 * (NCW + 4);
  static constexpr int VSEG = 0;
};

// Prepared tiles of one chunk-head in the workspace, in 16-byte units: of the LDS
// tiles of T~ hi, T~ lo and P, in that order, the part that the state pass reads
// (the operand rows of the lower-triangular block pairs): rows 0 .. 31, columns
// 0 .. 31 (4 units a row), then rows 32 .. 63, columns 0 .. 63 (8 units a row), in
// the tiles' permuted column order, strictly-upper blocks zero; then the chunk's
// gates beta_c, e^{gamma_c} and e^{gamma_last - gamma_c} (fp32, 64 each).  The
// rest of each tile (columns 32 .. 63 of rows 0 .. 31, and the row padding) stays
// zero in the state pass's LDS.  Chunk t of sequence s, v-head h is image (s TC +
// t) Hv + h, TC = ceil(T / C) (a sequence clamped into [0, T] has at most TC chunks).
constexpr int kTileUnits1 = 32 * 4 + 32 * 8;  // units of one tile
constexpr int kTileUnits = 3 * kTileUnits1;
constexpr int kGateUnits = 3 * C / 4;
constexpr int kTileImage = kTileUnits + kGateUnits;

// Element offset, from the tile's base, of unit e (0 .. kTileUnits1 - 1) of a tile's
// part of an image.
__device__ __forceinline__ int tile_unit_off(int e) {
  return e < 128 ? (e >> 2) * TSTR + 8 * (e & 3) : (32 + ((e - 128) >> 3)) * TSTR + 8 * ((e - 128) & 7);
}
constexpr int kMaxSortedSeqs = 1024;  // longest-first ordering up to this many sequences
constexpr int kMaxPersistList = 128;  // chains per workgroup of the persistent kernel
constexpr int kMaxPersistLpt = 64;    // batches of at most this many sequences get a longest-processing-time list

struct __align__(16) PrefillSmem {
  static constexpr int kParities = 2;  // chunk buffers in flight
  uint16_t K[2][C * KSTR];    // K chunk [c][perm(k)], by chunk parity
  uint16_t Q[2][C * KSTR];    // Q chunk [c][perm(k)]
  uint16_t Th[2][C * TSTR];   // T~ hi [c][perm(j)] (strictly-upper blocks stay 0)
  uint16_t Tl[2][C * TSTR];   // T~ lo
  uint16_t P[2][C * TSTR];    // P (bf16) [c][perm(j)] (strictly-upper blocks stay 0)
  uint16_t V[C * VSTR];       // V chunk [c][v], single-buffered (written after its last read)
  uint16_t Nh[NROWS * TSTR];  // N rows 16..63, hi [i - 16][perm(j)] (producers only; row block 0
  uint16_t Nl[NROWS * TSTR];  // of N is never an operand), lo
  float Nd[4 * NDB];          // diagonal 16x16 blocks of N (fp32, column-major: [block][col][row])
  float gam[2][C];            // gamma_c log2(e) (inclusive cumsum of the log2 gates), rounded
  float gaml[2][C];           // its rounding error (the sum is formed in fp64)
  float bet[2][C];            // beta_c
  float eg[2][C];             // e^{gamma_c}
  float dd[2][C];             // e^{gamma_last - gamma_c}
  int seq;                    // sequence handled by this workgroup
  int pseq[kMaxPersistList];  // persistent kernel: the sequences of the workgroup's chains, in order,
  int ps0[kMaxPersistList];   // their token ranges [ps0, ps1),
  int ps1[kMaxPersistList];
  int pcount;                 // and their number
  int plen[kMaxPersistLpt];   // persistent kernel, up to kMaxPersistLpt sequences: their lengths,
  int pstart[kMaxPersistLpt];  // starts and longest-first order (the list is formed while the
  int porder[kMaxPersistLpt];  // first chain runs)
  int sync[16];               // hand-off counters (enum SyncCounter)
  int spin_limit;             // kernels with testing hooks: polls before a hand-off wait gives up
  unsigned* aborts;           // kernels with testing hooks: optional count of waits that gave up
};

// Before a workgroup's first chunk its LDS tiles double as integer scratch: the
// longest-first ranking (pick_sequence) keeps up to kMaxSortedSeqs lengths in Nh, and
// the persistent kernel's boustrophedon lists keep lengths, starts and order of up to
// kMaxSortedSeqs sequences in V.
static_assert(kMaxSortedSeqs * sizeof(int) <= sizeof(PrefillSmem::Nh), "sequence lengths fit Nh");
static_assert(3 * kMaxSortedSeqs * sizeof(int) <= sizeof(PrefillSmem::V), "sequence lists fit V");

// The token-split state pass exchanges Y and the state's bf16 hi/lo parts through
// Nh/Nl (unused without producers): four 16-token blocks of Y and four 32-column
// blocks of the state, 16 and 32 bytes per lane.
constexpr int kYxBytes = 4 * 64 * 16 + 4 * 64 * 32;
static_assert(offsetof(PrefillSmem, Nh) % 16 == 0 &&
                  offsetof(PrefillSmem, Nl) == offsetof(PrefillSmem, Nh) + sizeof(PrefillSmem::Nh) &&
                  sizeof(PrefillSmem::Nh) + sizeof(PrefillSmem::Nl) >= kYxBytes,
              "Y exchange fits Nh and Nl");

// LDS of the prep kernel (two-kernel path): one chunk's buffers (the producers
// stage chunk t + 1 once the copier has written chunk t out) and no V, so that two
// workgroups share a CU.
struct __align__(16) PrepSmem {
  static constexpr int kParities = 1;
  uint16_t K[1][C * KSTR];
  uint16_t Q[1][C * KSTR];
  uint16_t Th[1][C * TSTR];
  uint16_t Tl[1][C * TSTR];
  uint16_t P[1][C * TSTR];
  uint16_t V[8];              // no V is staged (PrepVariant::VSEG = 0)
  uint16_t Nh[NROWS * TSTR];
  uint16_t Nl[NROWS * TSTR];
  float Nd[4 * NDB];
  float gam[1][C];
  float gaml[1][C];
  float bet[1][C];
  float eg[1][C];
  float dd[1][C];
  int sync[16];
  int spin_limit;
  unsigned* aborts;
};

// Gate arrays are copied to and from chunk images in 16-byte units, addressed from
// beta (gate_unit): 16-byte aligned, e^gamma and the update decay following it.
template <class Smem>
constexpr bool gates_follow_beta() {
  return offsetof(Smem, bet) % 16 == 0 && offsetof(Smem, eg) == offsetof(Smem, bet) + sizeof(Smem::bet) &&
         offsetof(Smem, dd) == offsetof(Smem, eg) + sizeof(Smem::eg) &&
         sizeof(Smem::bet) == Smem::kParities * C * sizeof(float);
}
static_assert(gates_follow_beta<PrefillSmem>() && gates_follow_beta<PrepSmem>(), "gate layout");

constexpr float kLog2e = 1.4426950408889634f;

// 2^{x} for x <= 0 (the hardware exp2, v_exp_f32).  Log gates are kept in log2
// units (gamma * log2(e)), so every decay e^{gamma_i - gamma_j} is one exp2.
__device__ __forceinline__ float exp2_le0(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x4 mfma(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Raw buffer resource over [base, base + bytes): a vector store whose byte offset
// (plus its size) reaches past `bytes` is dropped by the hardware, which replaces a
// per-lane branch around stores that may fall outside a chunk.  The third dword is
// the gfx9 raw-buffer format word (32-bit data format, no swizzle, no stride).
typedef __amdgpu_buffer_rsrc_t BufferRsrc;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ BufferRsrc buffer_rsrc(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, short(0), int(bytes), 0x00020000);
}
__device__ __forceinline__ void buffer_store16(u32x4 v, BufferRsrc r, int offset) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, offset, 0, 0);
}
__device__ __forceinline__ void buffer_store8(u32x2 v, BufferRsrc r, int offset) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, offset, 0, 0);
}

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1 (compile-time indices).
template <int I, int N, class Fn>
__device__ __forceinline__ void static_for_impl(Fn&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_impl<I + 1, N>(f);
  }
}
template <int N, class Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  static_for_impl<0, N>(f);
}

// Position of contraction index r (0..31) inside a 32-wide permuted block.
__device__ __forceinline__ int perm32(int r) { return ((r & 15) >> 2) * 8 + ((r >> 4) << 2) + (r & 3); }
__device__ __forceinline__ int perm(int x) { return (x & ~31) + perm32(x & 31); }

// K/Q tiles: element (r, q) (q = permuted column) lives in 16-byte slot
// (q / 8) ^ sigma(r) of row r.  sigma swaps bits 1 and 2 of r (and keeps bits 0
// and 3): eight consecutive rows then hit eight different slots (row-operand
// reads are conflict-free), and the four rows of a transposed read split over
// two slot ranges.
__device__ __forceinline__ int kq_sigma(int r) { return (r & 9) | ((r & 2) << 1) | ((r & 4) >> 1); }
__device__ __forceinline__ int kq_off(int r, int q) { return r * KSTR + (((q >> 3) ^ kq_sigma(r)) << 3) + (q & 7); }

// Operand row of a K/Q tile: rows row0 + lane%16, contraction block ks.
__device__ __forceinline__ uint4 frag_kq(const uint16_t* tile, int row0, int ks, int lane) {
  return *reinterpret_cast<const uint4*>(tile + kq_off(row0 + (lane & 15), 32 * ks + 8 * (lane >> 4)));
}

// Operand row: rows row0 + lane%16, contraction block ks (32 wide), from a tile
// stored with permuted columns.
__device__ __forceinline__ uint4 frag(const uint16_t* tile, int stride, int row0, int ks, int lane) {
  return *reinterpret_cast<const uint4*>(tile + (row0 + (lane & 15)) * stride + 32 * ks + 8 * (lane >> 4));
}

__device__ __forceinline__ uint2 read_tr(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

// Four rows k0 + 4g .. +3 of column col0 + lane%16 of a row-major tile whose
// columns are perm-ordered (groups of 4 columns stay contiguous).  In each
// 16-lane group, lane j reads 4 contiguous columns of row k0 + 4g + j/4; the
// transpose read hands lane i element i of each of those rows.
__device__ __forceinline__ uint2 col4_tr(const uint16_t* tile, int stride, int k0, int col0, int lane) {
  const int j = lane & 15, g = lane >> 4;
  return read_tr(tile + (k0 + 4 * g + (j >> 2)) * stride + perm(col0 + 4 * (j & 3)));
}


// Operand column of the K tile for the state update: column 16 kt + lane%16 (of
// the unpermuted k index), contraction rows 32 ks + kappa(g, s), as two
// transpose reads of 4 rows (k0 = 32 ks, then k0 + 16).  In 16-lane group g lane
// j reads 4 contiguous columns of row k0 + rl, rl = 4 g + j / 4, namely element
//   kq_off(k0 + rl, perm(16 kt + 4 (j & 3))),
// and perm(16 kt + 4 (j & 3)) = 32 (kt / 2) + 8 (j & 3) + 4 (kt & 1), so with
// s = sigma(rl) the offset is
//   (k0 + rl) KSTR + 32 ((kt / 2) ^ (s >> 2)) + 8 ((j & 3) ^ (s & 3)) + 4 (kt & 1):
// four lane bases (one per kt / 2) plus compile-time offsets.
struct KtBases {
  int b[4];
};
__device__ __forceinline__ KtBases kt_bases(int lane) {
  const int j = lane & 15, rl = 4 * (lane >> 4) + (j >> 2), sl = kq_sigma(rl);
  const int l0 = rl * KSTR + 8 * ((j & 3) ^ (sl & 3));
  KtBases r;
#pragma unroll
  for (int m = 0; m < 4; ++m) r.b[m] = l0 + 32 * (m ^ (sl >> 2));
  return r;
}
template <int KS, int KT>
__device__ __forceinline__ uint4 frag_tr_k_at(const uint16_t* tile, const KtBases& kb) {
  const uint16_t* p = tile + kb.b[KT / 2] + 32 * KS * KSTR + 4 * (KT & 1);
  const uint2 a = read_tr(p), b = read_tr(p + 16 * KSTR);
  return uint4{a.x, a.y, b.x, b.y};
}

// B/A operand (bf16 hi parts) from two accumulator tiles stacked along the
// contraction dim.
__device__ __forceinline__ uint4 pack_hi(const f32x4& t0, const f32x4& t1) {
  return uint4{pack_bf16x2(t0[0], t0[1]), pack_bf16x2(t0[2], t0[3]), pack_bf16x2(t1[0], t1[1]),
               pack_bf16x2(t1[2], t1[3])};
}

// 16x16x16 MFMA (one 16-wide contraction block): lane l supplies A[l%16][4g..4g+3]
// and B[4g..4g+3][l%16], g = l/16 -- the lower half of the 32-wide convention.
__device__ __forceinline__ f32x4 mfma16(const uint2& a, const uint2& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0,
                                                   0, 0);
}

// The residuals t - hi(t) of four fp32 values per lane, given their bf16 hi parts
// packed as a 16x16x16 B operand (lane l, slot s: B[4g + s][l%16]), formed on the
// matrix pipe: D = t + (-I) hi(t) with t as the accumulator, which lane l holds as
// D[4g + s][l%16] -- the same (lane, slot) for every element, so this is an
// elementwise t - hi(t).  Each element has one nonzero product and its exact result
// is representable, so the residual is exact (as the fp32 subtraction would be),
// and the wave issues one MFMA instead of eight VALU instructions.  -I as the A
// operand (lane l: row l%16, contraction 4g + s) has its one nonzero, bf16 -1, in
// slot l%4 when g == (l%16)/4.
__device__ __forceinline__ f32x4 residual4(const f32x4& t, const uint2& hi) {
  const uint32_t l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const uint32_t w = (l >> 4) == ((l & 15) >> 2) ? (0xbf80u << (16 * (l & 1))) : 0u;
  const uint2 neg_identity = (l & 2) ? uint2{0u, w} : uint2{w, 0u};
  return mfma16(neg_identity, hi, t);
}

// bf16 hi parts (round to nearest even) and lo parts (the residual, rounded) of
// two stacked accumulator tiles (B/A operands, as pack_hi) or of one.
__device__ __forceinline__ void split_pack(const f32x4& t0, const f32x4& t1, uint4& hi, uint4& lo) {
  hi = pack_hi(t0, t1);
  const f32x4 r0 = residual4(t0, uint2{hi.x, hi.y}), r1 = residual4(t1, uint2{hi.z, hi.w});
  lo = uint4{pack_bf16x2(r0[0], r0[1]), pack_bf16x2(r0[2], r0[3]), pack_bf16x2(r1[0], r1[1]),
             pack_bf16x2(r1[2], r1[3])};
}
__device__ __forceinline__ void split4(const f32x4& t, uint2& hi, uint2& lo) {
  hi = uint2{pack_bf16x2(t[0], t[1]), pack_bf16x2(t[2], t[3])};
  const f32x4 r = residual4(t, hi);
  lo = uint2{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
}

__device__ __forceinline__ int64_t load_cu(const void* cu, int is64, int i) {
  return is64 ? static_cast<const int64_t*>(cu)[i] : int64_t(static_cast<const int32_t*>(cu)[i]);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_or_zero(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, true));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_or_zero_f64(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0, uint32_t(u), CTRL, ROW_MASK, 0xF, true);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0, uint32_t(u >> 32), CTRL, ROW_MASK, 0xF, true);
  return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
}

// Inclusive prefix sum over the 64 lanes of a wavefront with DPP: shifts by
// 1, 2, 4, 8 inside each 16-lane row, then lane 15 of rows 0 / 2 into rows 1 / 3
// (row_bcast:15) and lane 31 into rows 2 and 3 (row_bcast:31).  The sum runs in
// fp64 and is returned as a pair hi + lo of floats (lo = the rounding error of
// hi): the decays e^{gamma_i - gamma_j} are formed from differences of these
// sums, and with fast decay the sums reach 1e5 in magnitude while a difference
// that matters (one that does not underflow to zero) is below 1e2 -- a plain
// fp32 difference would carry the sums' rounding error, up to about 1e-2.
__device__ __forceinline__ float wave_inclusive_scan2(float x, float& lo) {
  double d = x;
  d += dpp_or_zero_f64<0x111, 0xF>(d);
  d += dpp_or_zero_f64<0x112, 0xF>(d);
  d += dpp_or_zero_f64<0x114, 0xF>(d);
  d += dpp_or_zero_f64<0x118, 0xF>(d);
  d += dpp_or_zero_f64<0x142, 0xA>(d);
  d += dpp_or_zero_f64<0x143, 0xC>(d);
  const float hi = float(d);
  lo = float(d - double(hi));
  return hi;
}

// gamma_i - gamma_j from the pairs (hi, lo) of the compensated scan.  The hi
// difference is exact whenever it is small against the sums (Sterbenz), so the
// result is accurate to fp32 precision of the difference itself.
__device__ __forceinline__ float gamma_diff(float hi_i, float lo_i, float hi_j, float lo_j) {
  return (hi_i - hi_j) + (lo_i - lo_j);
}

// Log-space decay in log2 units, -exp(A_log) * softplus(a + dt_bias) * log2(e)
// (torch threshold 20), with the hardware exp2/log2; neg_decay = -exp(A_log).
// log2(1 + 2^y) is softplus(x) * log2(e) with y = x log2(e), so no conversion
// back to natural units is needed.  For very negative arguments log2(1 + 2^y)
// loses its relative accuracy but stays within ~2e-7 absolutely.
__device__ __forceinline__ float fast_log2_gate(float neg_decay, float x) {
  const float y = x * kLog2e;
  return neg_decay * (x > 20.f ? y : __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(y)));
}

__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// Sum over the four 16-lane rows of a wavefront (lanes j, j+16, j+32, j+48):
// the row swaps pair rows (0,1), (2,3), then the two halves.
__device__ __forceinline__ float sum_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Orders this wave's LDS writes before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace

// Waves on this device whose hand-off wait gave up (see wait_count), since the
// library was loaded or the count was last reset; read by prefill_giveups.
__device__ unsigned int gdn_prefill_giveup_count;

namespace {

// Hand-off between the two roles: monotonically increasing LDS counters.  A wave
// signals by adding 1 after its earlier LDS accesses (release: see signal_count); a
// waiter polls until the count reaches its target (acquire).
enum SyncCounter {
  kReady = 0,     // chunk handed over to the consumers (4 a chunk; pipelined: its T~ and P, NS + 2)
  kVFree = 1,     // consumers read the chunk's V
  kConsumed = 2,  // consumers done with the chunk's buffers
  kPPhase = 3,    // four producers: their step barriers; pipelined: solve and N tiles done (3 a chunk)
  kAbort = 4,     // a wait gave up
  kDiagN = 5,     // diagonal N tiles formed (4 a chunk)
  kX32 = 6,       // off-diagonal block X32 stored
  kStaged = 7,    // pipelined: the chunk's K/Q staged and its gates stored (NS + 1 a chunk)
  kNRead = 8,     // pipelined: the left off-diagonal wave read its N operands
  kVStaged = 9,   // pipelined: the chunk's V staged (NS a chunk)
  kList = 10,     // persistent kernel: the workgroup's chain list is complete (1)
  kYx = 11,       // token-split state pass: a consumer wave stored its block of Y (4 a chunk)
  kSx = 12        // token-split state pass: a consumer wave stored its state columns (4 a chunk, 4 at start)
};
constexpr int kSpinLimit = 1 << 21;  // default polls (about 70 ms) before a wait gives up

// Every hand-off publishes LDS data (or releases LDS reads) to waves of the same
// workgroup, through an LDS counter.  The LDS performs a CU's operations in one
// order, and a wave's own LDS operations in the order the wave issues them, so the
// increment is performed after every LDS write or read the wave issued before it,
// and a waiter that sees the count issues its reads after that.  No wait for the
// wave's outstanding LDS operations is needed before the increment (a workgroup-
// scope release fence would add one, s_waitcnt lgkmcnt(0), which stalls the
// signalling wave until its last writes land); the compiler-level fences keep the
// program order.  Nothing is published through these counters in global memory.
template <class Smem>
__device__ __forceinline__ void signal_count(Smem& sm, int which, int lane) {
  (void)lane;
  // One LDS add from lane 0, with exec set to that lane inside one asm block rather
  // than by a branch, so that the surrounding arithmetic is still scheduled as one
  // block.  Every caller runs with the whole wave active.  The block writes no SCC
  // (s_mov only), and the compiler does not count its LDS operation in its waits, which
  // can only make those stricter (a wave's LDS operations complete in order).
  typedef __attribute__((address_space(3))) int lds_int;
  const uint32_t addr = uint32_t(reinterpret_cast<uintptr_t>((lds_int*)(&sm.sync[which])));
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %0, exec\n\t"
      "s_mov_b64 exec, 1\n\t"
      "ds_add_u32 %1, %2\n\t"
      "s_mov_b64 exec, %0"
      : "=&s"(saved)
      : "v"(addr), "v"(1)
      : "memory");
}

// Waits until counter `which` reaches `target`.  Every wait is bounded: if one
// ever gives up (which only a logic error, or the testing hooks of PrefillArgs,
// can cause), it raises kAbort, and all later waits return at once, so the
// workgroup still finishes instead of hanging.  The wave that gives up adds 1 to
// gdn_prefill_giveup_count (a global atomic from one lane), and the workgroup
// writes NaN to every output element and state element it owns (and the prep
// kernel NaN images), so wrong results never look valid.  Production kernels give
// up after kSpinLimit polls; kernels built with the hooks after sm.spin_limit
// polls, also counting each give-up in sm.aborts if set.
template <bool kHooks, class Smem>
__device__ __forceinline__ void wait_count(Smem& sm, int which, int target) {
  if (__hip_atomic_load(&sm.sync[which], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    for (int it = 0;; ++it) {
      __builtin_amdgcn_s_sleep(1);
      if (__hip_atomic_load(&sm.sync[which], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
      if (__hip_atomic_load(&sm.sync[kAbort], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0) break;
      if (it >= (kHooks ? sm.spin_limit : kSpinLimit)) {
        __hip_atomic_store(&sm.sync[kAbort], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) == 0) {
          __hip_atomic_fetch_add(&gdn_prefill_giveup_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if constexpr (kHooks) {
            unsigned* aborts = sm.aborts;
            if (aborts) __hip_atomic_fetch_add(aborts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        break;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// wait_count for counter `a`, reading counter `b` in the same LDS round trip:
// returns whether `b` had reached `tb` then, so that a later wait for it can be
// skipped (the acquire that ends this wait covers both).
template <bool kHooks, class Smem>
__device__ __forceinline__ bool wait_count_peek(Smem& sm, int a, int ta, int b, int tb) {
  const int va = __hip_atomic_load(&sm.sync[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  const int vb = __hip_atomic_load(&sm.sync[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  const bool b_ok = __builtin_amdgcn_readfirstlane(int(vb >= tb)) != 0;
  if (__builtin_amdgcn_readfirstlane(int(va >= ta)) != 0) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  } else {
    wait_count<kHooks>(sm, a, ta);
  }
  return b_ok;
}

template <class Smem>
__device__ __forceinline__ bool aborted(Smem& sm) {
  return __hip_atomic_load(&sm.sync[kAbort], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
}

constexpr uint32_t kNaNx2 = 0x7fc07fc0u;  // two bf16 quiet NaNs


// The parity-selected LDS buffers of one chunk.
struct ChunkBufs {
  uint16_t* K;
  uint16_t* Q;
  uint16_t* Th;
  uint16_t* Tl;
  uint16_t* P;
  float* gam;
  float* gaml;
  float* bet;
  float* eg;
  float* dd;
};

template <class Smem>
__device__ __forceinline__ ChunkBufs chunk_bufs(Smem& sm, int b) {
  b %= Smem::kParities;
  return ChunkBufs{sm.K[b],   sm.Q[b],   sm.Th[b],  sm.Tl[b], sm.P[b],
                   sm.gam[b], sm.gaml[b], sm.bet[b], sm.eg[b], sm.dd[b]};
}

// ---------------------------------------------------------------------------
// Producer side (waves NCW .. NCW+3)
// ---------------------------------------------------------------------------

// Tiles of N and P from the staged K and Q (16x16 tiles, 4 MFMAs each).
//   kind 1: off-diagonal block (I, J), I > J, of N (bf16 hi/lo), from tile
//           K_J K_I^T so that a lane holds 4 consecutive columns of one row
//   kind 2: block (I, J), J <= I, of P, from tile K_J Q_I^T
struct TileJob {
  int kind, I, J;
};

__device__ __forceinline__ f32x4 ld4(const float* p) {
  const float4 x = *reinterpret_cast<const float4*>(p);
  return f32x4{x.x, x.y, x.z, x.w};
}

// Branch-free epilogues: gamma is non-increasing along the chunk, so every
// exponent kept is <= 0; the masked ones are clamped to 0 before the select.
template <class Smem>
__device__ __forceinline__ void tile_epilogue(Smem& sm, const ChunkBufs& cb, const TileJob t, const f32x4& acc,
                                              float scale, int lane) {
  const int g = lane >> 4, n16 = lane & 15;
  if (t.kind == 1) {
    // acc[i] = k_c . k_r, c = 16J + 4g + i, r = 16I + n16  ->  N[r][c]  (r > c)
    const int r = 16 * t.I + n16;
    const float gr = cb.gam[r], grl = cb.gaml[r], br = cb.bet[r];
    const f32x4 gcv = ld4(cb.gam + 16 * t.J + 4 * g), gcl = ld4(cb.gaml + 16 * t.J + 4 * g);
    f32x4 x;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = br * exp2_le0(fminf(gamma_diff(gr, grl, gcv[i], gcl[i]), 0.f)) * acc[i];
    uint2 hi, lo;
    split4(x, hi, lo);
    const int pos = (r - 16) * TSTR + perm(16 * t.J + 4 * g);
    *reinterpret_cast<uint2*>(sm.Nh + pos) = hi;
    *reinterpret_cast<uint2*>(sm.Nl + pos) = lo;
  } else {
    // acc[i] = k_j . q_c, j = 16J + 4g + i, c = 16I + n16  ->  P[c][j]  (j <= c),
    // with the output scale folded in
    const int c = 16 * t.I + n16;
    const float gc = cb.gam[c], gcl = cb.gaml[c];
    const f32x4 gj = ld4(cb.gam + 16 * t.J + 4 * g), gjl = ld4(cb.gaml + 16 * t.J + 4 * g);
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = exp2_le0(fminf(gamma_diff(gc, gcl, gj[i], gjl[i]), 0.f)) * (acc[i] * scale);
      pv[i] = 16 * t.J + 4 * g + i <= c ? x : 0.f;
    }
    *reinterpret_cast<uint2*>(cb.P + c * TSTR + perm(16 * t.J + 4 * g)) =
        uint2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
  }
}

template <int NJ, class Smem>
__device__ __forceinline__ void run_tiles(Smem& sm, const ChunkBufs& cb, const TileJob (&jobs)[NJ], float scale,
                                          int lane) {
  f32x4 acc[NJ];
#pragma unroll
  for (int t = 0; t < NJ; ++t) acc[t] = zero4();
  uint4 a[NJ][4], b[NJ][4];  // all operands first: one round of LDS latency
#pragma unroll
  for (int t = 0; t < NJ; ++t) {
    const TileJob j = jobs[t];
    const int arow = 16 * j.J;
    const uint16_t* btile = j.kind == 2 ? cb.Q : cb.K;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      a[t][ks] = frag_kq(cb.K, arow, ks, lane);
      b[t][ks] = frag_kq(btile, 16 * j.I, ks, lane);
    }
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int t = 0; t < NJ; ++t) acc[t] = mfma(a[t][ks], b[t][ks], acc[t]);
#pragma unroll
  for (int t = 0; t < NJ; ++t) tile_epilogue(sm, cb, jobs[t], acc[t], scale, lane);
}

// The four diagonal blocks of T~, D_I = (I + N_II)^-1.  diag_tiles forms N_II
// from the tiles K_I K_I^T (scaled as in the off-diagonal epilogue) for blocks
// I0 .. I1-1, stored column-major; diag_solve (one wavefront, all four blocks)
// then has lane (r, j) = (lane/16, lane%16) invert block r, column j,
// x = D_r[:, j], by right-looking forward substitution:
//   x_m = delta_mj - a_m,  a_i += N[i][m] x_m  for i > m
// (for m < j every term is zero, so x_m = 0 there).  The column of N needed at
// step m is one broadcast read per four rows; no cross-lane traffic.
template <int I0, int I1, class Smem>
__device__ __forceinline__ void diag_tiles(Smem& sm, const ChunkBufs& cb, int lane) {
  const int g = lane >> 4, n16 = lane & 15;
  {
    f32x4 acc[4];
#pragma unroll
    for (int I = I0; I < I1; ++I) {
      uint4 kf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kf[ks] = frag_kq(cb.K, 16 * I, ks, lane);
      acc[I] = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc[I] = mfma(kf[ks], kf[ks], acc[I]);
    }
    // acc[I][i] = k_r . k_c, r = 16I + 4g + i, c = 16I + n16 -> N[r][c] for r > c
    // (entries with r <= c are never read).
#pragma unroll
    for (int I = I0; I < I1; ++I) {
      const float gc = cb.gam[16 * I + n16], gcl = cb.gaml[16 * I + n16];
      const f32x4 gr = ld4(cb.gam + 16 * I + 4 * g), grl = ld4(cb.gaml + 16 * I + 4 * g);
      const f32x4 br = ld4(cb.bet + 16 * I + 4 * g);
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = br[i] * exp2_le0(fminf(gamma_diff(gr[i], grl[i], gc, gcl), 0.f)) * acc[I][i];
      *reinterpret_cast<f32x4*>(sm.Nd + I * NDB + n16 * 16 + 4 * g) = x;
    }
  }
}

template <class Smem>
__device__ __forceinline__ void diag_solve(Smem& sm, const ChunkBufs& cb, int lane) {
  const int r = lane >> 4, j = lane & 15;
  const float* nb = sm.Nd + r * NDB;
  // Columns are read kColAhead steps ahead of their use.
  constexpr int kColAhead = 4;
  f32x4 colv[15][4];
#pragma unroll
  for (int m = 0; m < kColAhead; ++m)
#pragma unroll
    for (int q = (m + 1) / 4; q < 4; ++q) colv[m][q] = ld4(nb + m * 16 + 4 * q);
  float a[16], x[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    x[m] = (m == j) ? 1.f : (m == 0 ? 0.f : -a[m]);
    if (m + kColAhead < 15) {
#pragma unroll
      for (int q = (m + kColAhead + 1) / 4; q < 4; ++q)
        colv[m + kColAhead][q] = ld4(nb + (m + kColAhead) * 16 + 4 * q);
    }
    if (m < 15) {
#pragma unroll
      for (int q = (m + 1) / 4; q < 4; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * q + e;
          if (i > m) a[i] = m == 0 ? colv[m][q][e] * x[0] : fmaf(colv[m][q][e], x[m], a[i]);
        }
      }
    }
  }
  // rows 16r + i, column 16r + j of T~
  const int colp = perm(16 * r + j);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint2 hi, lo;
    split4(f32x4{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]}, hi, lo);
    const uint32_t h4[4] = {hi.x, hi.x >> 16, hi.y, hi.y >> 16}, l4[4] = {lo.x, lo.x >> 16, lo.y, lo.y >> 16};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cb.Th[(16 * r + 4 * q + e) * TSTR + colp] = uint16_t(h4[e]);
      cb.Tl[(16 * r + 4 * q + e) * TSTR + colp] = uint16_t(l4[e]);
    }
  }
}

struct Pair2 {  // bf16 hi / lo parts of a 16x16x16 operand
  uint2 h, l;
};

// acc += A B, both as hi/lo pairs (three passes).
__device__ __forceinline__ f32x4 mul3_16(f32x4 acc, const Pair2& a, const Pair2& b) {
  acc = mfma16(a.h, b.h, acc);
  acc = mfma16(a.h, b.l, acc);
  acc = mfma16(a.l, b.h, acc);
  return acc;
}

// B operand from an fp32 accumulator tile.
__device__ __forceinline__ Pair2 acc_b(const f32x4& t) {
  Pair2 r;
  split4(t, r.h, r.l);
  return r;
}

// A operand of the 16x16 block (I, J) of a hi/lo tile pair with permuted columns
// (row0 = first row held by the tiles).
__device__ __forceinline__ Pair2 block_a(const uint16_t* th, const uint16_t* tl, int row0, int I, int J, int lane) {
  const int off = (16 * I - row0 + (lane & 15)) * TSTR + perm(16 * J + 4 * (lane >> 4));
  return Pair2{*reinterpret_cast<const uint2*>(th + off), *reinterpret_cast<const uint2*>(tl + off)};
}

// B operand of the diagonal block D_J of T~.
__device__ __forceinline__ Pair2 diag_b(const ChunkBufs& cb, int J, int lane) {
  return Pair2{col4_tr(cb.Th, TSTR, 16 * J, 16 * J, lane), col4_tr(cb.Tl, TSTR, 16 * J, 16 * J, lane)};
}

// Writes an off-diagonal block X_IJ (accumulator layout) to Th/Tl.
__device__ __forceinline__ void store_block(const ChunkBufs& cb, const f32x4& X, int I, int J, int lane) {
  const int g = lane >> 4, col = perm(16 * J + (lane & 15));
  uint2 hi, lo;
  split4(X, hi, lo);
  const uint32_t h4[4] = {hi.x, hi.x >> 16, hi.y, hi.y >> 16}, l4[4] = {lo.x, lo.x >> 16, lo.y, lo.y >> 16};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    cb.Th[(16 * I + 4 * g + i) * TSTR + col] = uint16_t(h4[i]);
    cb.Tl[(16 * I + 4 * g + i) * TSTR + col] = uint16_t(l4[i]);
  }
}

// X_IJ = D_I (-G): written to Th/Tl and returned.
__device__ __forceinline__ f32x4 finish_block(const ChunkBufs& cb, const f32x4& G, const Pair2& dI, int I, int J,
                                              int lane) {
  const f32x4 X = mul3_16(zero4(), dI, acc_b(-G));
  store_block(cb, X, I, J, lane);
  return X;
}

// Off-diagonal blocks of T~, as a 2x2 block inverse over the 32x32 halves:
//   T~ = [[A^-1, 0], [-B^-1 C A^-1, B^-1]] with
//   A^-1 = [[D0, 0], [X10, D1]],  B^-1 = [[D2, 0], [X32, D3]],  C = [[N20, N21], [N30, N31]],
//   X10 = -D1 N10 D0,  X32 = -D3 N32 D2,  M = C A^-1,  [[X20, X21], [X30, X31]] = -B^-1 M.
// Two wavefronts share it.  Column 1 of M (N21 D1, N31 D1) does not need X10,
// so one wave forms X32, X21 and X31 (offdiag_right) while the other forms X10,
// X20 and X30 (offdiag_left); the left wave reads X32 back from T~ once the
// right wave has stored it (counter kX32).  Each wave reads all of its LDS
// operands before its first block store.
template <class Smem>
__device__ __forceinline__ void offdiag_right(Smem& sm, const ChunkBufs& cb, int t, int lane) {
  const Pair2 d1 = diag_b(cb, 1, lane), d2 = diag_b(cb, 2, lane);
  const Pair2 a2 = block_a(cb.Th, cb.Tl, 0, 2, 2, lane), a3 = block_a(cb.Th, cb.Tl, 0, 3, 3, lane);
  const Pair2 n21 = block_a(sm.Nh, sm.Nl, 16, 2, 1, lane), n31 = block_a(sm.Nh, sm.Nl, 16, 3, 1, lane),
              n32 = block_a(sm.Nh, sm.Nl, 16, 3, 2, lane);
  const f32x4 g32 = mul3_16(zero4(), n32, d2);
  const f32x4 m21 = mul3_16(zero4(), n21, d1);
  const f32x4 m31 = mul3_16(zero4(), n31, d1);
  finish_block(cb, g32, a3, 3, 2, lane);  // X32
  signal_count(sm, kX32, lane);
  const Pair2 x32t = acc_b(mul3_16(zero4(), acc_b(-g32), a3));  // A operand holding X32
  const Pair2 nm21 = acc_b(-m21), nm31 = acc_b(-m31);
  store_block(cb, mul3_16(zero4(), a2, nm21), 2, 1, lane);                           // X21
  store_block(cb, mul3_16(mul3_16(zero4(), x32t, nm21), a3, nm31), 3, 1, lane);      // X31
  (void)t;
}

template <bool kHooks, bool kSignalNRead = false, class Smem>
__device__ __forceinline__ void offdiag_left(Smem& sm, const ChunkBufs& cb, int t, int lane) {
  const Pair2 d0 = diag_b(cb, 0, lane);
  const Pair2 a1 = block_a(cb.Th, cb.Tl, 0, 1, 1, lane), a2 = block_a(cb.Th, cb.Tl, 0, 2, 2, lane),
              a3 = block_a(cb.Th, cb.Tl, 0, 3, 3, lane);
  const Pair2 n10 = block_a(sm.Nh, sm.Nl, 16, 1, 0, lane), n20 = block_a(sm.Nh, sm.Nl, 16, 2, 0, lane),
              n21 = block_a(sm.Nh, sm.Nl, 16, 2, 1, lane), n30 = block_a(sm.Nh, sm.Nl, 16, 3, 0, lane),
              n31 = block_a(sm.Nh, sm.Nl, 16, 3, 1, lane);
  // (Seven producers: the N tiles of the next chunk may be written once these reads
  // are done; the signal's release waits for them.)
  if constexpr (kSignalNRead) signal_count(sm, kNRead, lane);
  const f32x4 g10 = mul3_16(zero4(), n10, d0);
  const f32x4 p20 = mul3_16(zero4(), n20, d0);
  const f32x4 p30 = mul3_16(zero4(), n30, d0);
  const f32x4 x10 = finish_block(cb, g10, a1, 1, 0, lane);  // X10
  const Pair2 b10 = acc_b(x10);
  const Pair2 nm20 = acc_b(-mul3_16(p20, n21, b10));
  const Pair2 nm30 = acc_b(-mul3_16(p30, n31, b10));
  store_block(cb, mul3_16(zero4(), a2, nm20), 2, 0, lane);  // X20
  const f32x4 x30 = mul3_16(zero4(), a3, nm30);
  wait_count<kHooks>(sm, kX32, t + 1);  // X32 stored by the right wave
  const Pair2 x32 = block_a(cb.Th, cb.Tl, 0, 3, 2, lane);
  store_block(cb, mul3_16(x30, x32, nm20), 3, 0, lane);     // X30
}

// Global loads.  A CU streams about 48 KB of K, Q and V per chunk through its
// vector-memory pipe, and a wave that issues loads while that queue is full
// stalls until it drains.  The producers issue the next chunk's K/Q loads at
// the start of their middle step, while the consumers' retrieve (the heaviest
// LDS reader) runs, so the stall overlaps LDS work that would hold them up
// anyway.
//
// With NT threads sharing the K/Q rows of a chunk, thread pt (0..NT-1) owns K/Q
// segments pt + NT it: token pt/16 + (NT/16) it, columns 8 (pt%16) .. +7 (16
// consecutive threads read one 256-byte row); four producer waves (NT = 256) take
// tokens pt/16 + 16 it, it = 0..3.  Addresses are a wave-uniform chunk base (64-bit,
// scalar) plus a 32-bit lane offset that is fixed across chunks.
constexpr int NPROD = 256;  // producer threads (four waves)

template <int NT>
struct ProducerPrefetchT {
  static constexpr int RS = NT / 16;              // tokens between a thread's segments
  static constexpr int NIT = (C + RS - 1) / RS;   // segments per thread
  static_assert(NT % 64 == 0 && NT >= 64 && NT <= 256, "whole waves share the staging");
  uint4 k[NIT], q[NIT];
  uint16_t a, b;  // raw gate inputs of token pt (first wave only)
};
using ProducerPrefetch = ProducerPrefetchT<NPROD>;

struct LaneOffsets {
  int k, q;  // (pt/16) rows + 8 (pt%16) elements, in the K and Q row strides
  int ab;    // pt rows of the a/b [T, Hv] layout
};

template <int NT>
__device__ __forceinline__ void producer_prefetch(const PrefillArgs& p, int64_t cs, int clen, int h, int hq, int hk,
                                                  int pt, const LaneOffsets& lo, ProducerPrefetchT<NT>& f) {
  constexpr int RS = ProducerPrefetchT<NT>::RS;
  const uint16_t* kb = p.k + (cs * p.Hk + hk) * D;
  const uint16_t* qb = p.q + (cs * p.Hq + hq) * D;
#pragma unroll
  for (int it = 0; it < ProducerPrefetchT<NT>::NIT; ++it) {
    const int c = (pt >> 4) + RS * it;
    f.k[it] = f.q[it] = uint4{0u, 0u, 0u, 0u};
    if (c < clen) {
      f.k[it] = *reinterpret_cast<const uint4*>(kb + (lo.k + RS * it * p.Hk * D));
      f.q[it] = *reinterpret_cast<const uint4*>(qb + (lo.q + RS * it * p.Hq * D));
    }
  }
  if (pt < 64) {  // wave-uniform; the row index is clamped and padding masked when used
    const int off = pt < clen ? lo.ab : (clen - 1) * p.Hv;
    f.a = (p.a + cs * p.Hv + h)[off];
    f.b = (p.b + cs * p.Hv + h)[off];
  }
}

// The gates of token `lane` of a chunk (first producer wave, from the raw a/b
// values of its prefetch): the log2-gate prefix sum as an fp32 pair, beta,
// e^gamma and the update decay e^{gamma_last - gamma}.
struct ChunkGates {
  float gam, gaml, bet, eg, dd;
};

template <int NT>
__device__ __forceinline__ ChunkGates chunk_gates(const ProducerPrefetchT<NT>& f, int lane, int clen, float neg_decay,
                                                  float dt_bias) {
  const float lg = lane < clen ? fast_log2_gate(neg_decay, bf16_to_f32(f.a) + dt_bias) : 0.f;
  ChunkGates g;
  g.bet = lane < clen ? fast_sigmoid(bf16_to_f32(f.b)) : 0.f;
  g.gam = wave_inclusive_scan2(lg, g.gaml);
  const float glast = readlane_f(g.gam, clen - 1), glastl = readlane_f(g.gaml, clen - 1);
  g.eg = exp2_le0(g.gam);
  g.dd = exp2_le0(fminf(gamma_diff(glast, glastl, g.gam, g.gaml), 0.f));
  return g;
}

__device__ __forceinline__ void store_gates(const ChunkBufs& cb, const ChunkGates& g, int lane) {
  cb.gam[lane] = g.gam;
  cb.gaml[lane] = g.gaml;
  cb.bet[lane] = g.bet;
  cb.eg[lane] = g.eg;
  cb.dd[lane] = g.dd;
}

// Step 1 of a chunk: the prefetched K and Q rows into the chunk's tiles
// (permuted columns).
template <int NT>
__device__ __forceinline__ void stage_kq(const ChunkBufs& cb, const ProducerPrefetchT<NT>& f, int pt) {
  constexpr int RS = ProducerPrefetchT<NT>::RS;
#pragma unroll
  for (int it = 0; it < ProducerPrefetchT<NT>::NIT; ++it) {
    const int c = (pt >> 4) + RS * it, sg = pt & 15;
    if (RS * ProducerPrefetchT<NT>::NIT > C && c >= C) break;  // past the chunk (NT not dividing 1024)
    const int col0 = (8 * sg) & ~31, r0 = (8 * sg) & 31;
    const int pa = kq_off(c, col0 + perm32(r0)), pb = kq_off(c, col0 + perm32(r0 + 4));
    *reinterpret_cast<uint2*>(cb.K + pa) = uint2{f.k[it].x, f.k[it].y};
    *reinterpret_cast<uint2*>(cb.K + pb) = uint2{f.k[it].z, f.k[it].w};
    *reinterpret_cast<uint2*>(cb.Q + pa) = uint2{f.q[it].x, f.q[it].y};
    *reinterpret_cast<uint2*>(cb.Q + pb) = uint2{f.q[it].z, f.q[it].w};
  }
}

// Step 1 with the chunk's gates formed in place (first wave).
__device__ __forceinline__ void stage_kq_gates(const ChunkBufs& cb, const ProducerPrefetch& f, int pt, int pw, int lane,
                                               int clen, float neg_decay, float dt_bias) {
  stage_kq(cb, f, pt);
  if (pw == 0) store_gates(cb, chunk_gates(f, lane, clen, neg_decay, dt_bias), lane);
}

// Unit g of a chunk's gates (beta, e^gamma, e^{gamma_last - gamma}; 16 units each),
// as an offset from beta, so that the address stays a known LDS address.
template <class Smem>
__device__ __forceinline__ float* gate_unit(const ChunkBufs& cb, int g) {
  return cb.bet + (g >> 4) * (Smem::kParities * C) + 4 * (g & 15);
}

// Producer thread pt's share of a chunk's T~ hi, T~ lo and P tiles (the parts of
// their LDS tiles that the state pass reads) and gates to the chunk's image in the
// workspace; NaN images once a hand-off wait of the workgroup gave up.  The gates go
// out from the first wave, which stores the next chunk's gates after this copy.
template <class Smem>
__device__ __forceinline__ void copy_tiles_out(const ChunkBufs& cb, u32x4* image, int pt, bool poison) {
  constexpr int NT1 = kTileUnits1;
  constexpr int NIT = (kTileUnits + NPROD - 1) / NPROD;
  constexpr u32x4 nan4 = u32x4{kNaNx2, kNaNx2, kNaNx2, kNaNx2};
  // All LDS reads first (one round of latency), then the stores; units past the
  // tiles (last round) re-read the last unit and store nothing.
  u32x4 v[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int e = pt + it * NPROD < kTileUnits ? pt + it * NPROD : kTileUnits - 1;
    const uint16_t* src = e < NT1       ? cb.Th + tile_unit_off(e)
                          : e < 2 * NT1 ? cb.Tl + tile_unit_off(e - NT1)
                                        : cb.P + tile_unit_off(e - 2 * NT1);
    v[it] = *reinterpret_cast<const u32x4*>(src);
  }
  const u32x4 gv = pt < kGateUnits ? *reinterpret_cast<const u32x4*>(gate_unit<Smem>(cb, pt)) : nan4;
#pragma unroll
  for (int it = 0; it < NIT; ++it)
    if (pt + it * NPROD < kTileUnits) image[pt + it * NPROD] = poison ? nan4 : v[it];
  if (pt < kGateUnits) image[kTileUnits + pt] = poison ? nan4 : gv;
}

// Persistent kernel: the number of chains in the workgroup's list, and the first
// chain at or after position k that has tokens (chain_count if none).
template <class Smem>
__device__ __forceinline__ int chain_count(Smem& sm) {
  return min(sm.pcount, kMaxPersistList);
}

template <class Smem>
__device__ __forceinline__ int next_chain(Smem& sm, int k) {
  const int n = chain_count(sm);
  while (k < n && sm.ps1[k] <= sm.ps0[k]) ++k;
  return k;
}

// The producer loop: chunk t is prepared into the buffers of parity t & 1 (of
// Smem::kParities) once the consumers are done with the chunk that used them last
// (chunk t - 2 with two parities).  The four producer waves meet twice per chunk
// (after staging; after the tiles and diagonal blocks) on their own counter; the
// chunk is handed over when all four are done.  V is staged for the workgroup's
// state rows [row0, row0 + ROWS) only.
// With V::kCopy (the prep kernel, no consumers) the producers also write each
// chunk's tiles to images (chunk t of the run at images + t Hv kTileImage): chunk
// t - 1's in step 1 of tick t, once all four waves have handed it over (so also
// done with its K and Q, which the staging overwrites), and before the staging
// barrier, after which tick t writes the same tiles; the first wave copies the
// gates out before it stores the next chunk's.
template <class V, class Smem>
__device__ __forceinline__ void producer_loop(Smem& sm, const PrefillArgs& p, int64_t s0, int64_t s1,
                                              int nchunks, int h, int hq, int hk, int row0, int pw, int lane0,
                                              u32x4* images = nullptr) {
  constexpr int NVIT = V::VSEG > 0 ? (V::VSEG + NPROD - 1) / NPROD : 1;  // V segments per producer thread
  const int pt = pw * 64 + lane0;
  const float neg_decay = -expf(p.A_log[h]);
  const float dt_bias = p.dt_bias[h];
  const LaneOffsets lo = {(pt >> 4) * p.Hk * D + 8 * (pt & 15), (pt >> 4) * p.Hq * D + 8 * (pt & 15), pt * p.Hv};
  // V slice: segment pt + 256 it is token c, columns row0 + 8 sg .. +7.
  int voff[NVIT], vrow[NVIT];
#pragma unroll
  for (int it = 0; it < NVIT; ++it) {
    const int seg = pt + it * NPROD, c = seg / (V::ROWS / 8), sg = seg % (V::ROWS / 8);
    vrow[it] = seg < V::VSEG ? c : C;  // C: no segment
    voff[it] = c * p.Hv * D + 8 * sg;
  }
  static_assert(V::NP == 4 && !V::kPipelined, "pipelined producers run producer_loop_split");
  // The persistent kernel runs the chains of the workgroup's list (chain k covers
  // tokens [s0, s1)) as one stream of chunks; u counts the chunks of the stream and
  // indexes the hand-offs and the buffer parities (u = t otherwise).  Chain 0
  // (the longest of the list) is known before the rest of the list, which is
  // waited for (kList) where the stream first looks past a chain.
  int k = 0;
  bool listed = false;
  if constexpr (V::kPersist) {
    s0 = sm.ps0[0];
    s1 = sm.ps1[0];
    nchunks = int((s1 - s0 + C - 1) / C);
    if (nchunks == 0) return;  // the longest chain is empty: so are the others
  }
  ProducerPrefetch f;
  uint4 fv[NVIT];
  producer_prefetch(p, s0, int(s1 - s0 < C ? s1 - s0 : C), h, hq, hk, pt, lo, f);
  // The first wave forms each chunk's gates one tick ahead (chunk t + 1's in step 3
  // of tick t, where it has slack) and stores them with the chunk's K and Q.
  ChunkGates gts = {0.f, 0.f, 0.f, 0.f, 0.f};
  if (pw == 0) gts = chunk_gates(f, lane0, int(s1 - s0 < C ? s1 - s0 : C), neg_decay, dt_bias);

  int u = 0;
  for (;;) {
  for (int t = 0; t < nchunks; ++t, ++u) {
    // The lane index is re-materialised opaquely each tick so that lane-dependent
    // LDS addresses are recomputed in the loop rather than hoisted and spilled.
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int64_t cs = s0 + int64_t(t) * C;
    const int clen = int(s1 - cs < C ? s1 - cs : C);
    // The next chunk: this chain's, or (persistent) the next chain's first.
    int64_t ncs = cs + C;
    int nclen = int(s1 - ncs < C ? s1 - ncs : C);
    bool has_next = ncs < s1;
    if constexpr (V::kPersist) {
      if (!has_next) {
        if (!listed) {
          wait_count<V::kHooks>(sm, kList, 1);
          listed = true;
        }
        const int nk = next_chain(sm, k + 1);
        if (nk < chain_count(sm)) {
          has_next = true;
          ncs = sm.ps0[nk];
          nclen = int(sm.ps1[nk] - ncs < C ? sm.ps1[nk] - ncs : C);
        }
      }
    }
    const ChunkBufs cb = chunk_bufs(sm, u & 1);
    // The buffers of chunk u - kParities (the same ones) consumed.
    constexpr int kPar = Smem::kParities;
    if (u >= kPar) wait_count<V::kHooks>(sm, kConsumed, V::NCW * (u - kPar + 1));
    if constexpr (V::kCopy) {
      if (t >= 1) wait_count<V::kHooks>(sm, kReady, 4 * t);  // chunk t - 1 handed over by all four waves
    }

    // 1: stage K/Q (permuted columns), gates
    stage_kq(cb, f, pt);
    if constexpr (V::kCopy) {
      // Chunk t - 1's tiles out, after the staging: its stores are counted with the
      // loads, and the staging's wait for its registers would wait for them too.
      if (t >= 1)
        copy_tiles_out<Smem>(chunk_bufs(sm, (t - 1) & 1), images + int64_t(t - 1) * p.Hv * kTileImage, pt, aborted(sm));
    }
    if (pw == 0) store_gates(cb, gts, lane);
    // The V slice of this chunk into registers; staged at the end of the tick,
    // after the consumers' last read of the previous chunk's V.
    {
      const uint16_t* vb = p.v + (cs * p.Hv + h) * D + row0;
#pragma unroll
      for (int it = 0; it < NVIT; ++it) {
        fv[it] = uint4{0u, 0u, 0u, 0u};
        if (vrow[it] < clen) fv[it] = *reinterpret_cast<const uint4*>(vb + voff[it]);
      }
    }
    signal_count(sm, kPPhase, lane);
    wait_count<V::kHooks>(sm, kPPhase, 4 * (2 * u + 1));  // all of K/Q/gates staged
    // The rest of the chunk is the longer chain: producer waves go ahead of the
    // consumer wave sharing the SIMD.
    __builtin_amdgcn_s_setprio(1);

    // 2: the next chunk's K/Q loads; diagonal N tiles (the solve waits for
    // them); then the diagonal blocks of T~ (wave 0) or the off-diagonal N tiles
    // and two P tiles each (the others, in the solve's shadow: P does not depend
    // on T~).
    // Split variants (few chains, a light consumer) put the solve first: the
    // other waves issue their loads after their diagonal tile, the solve wave
    // after its solve.
    constexpr bool kSolveFirst = V::F > 1;
    if (!kSolveFirst && has_next) producer_prefetch(p, ncs, nclen, h, hq, hk, pt, lo, f);
    switch (pw) {
      case 0:
        diag_tiles<0, 1>(sm, cb, lane);
        signal_count(sm, kDiagN, lane);
        wait_count<V::kHooks>(sm, kDiagN, 4 * (u + 1));
        diag_solve(sm, cb, lane);
        break;
      case 1: {
        diag_tiles<1, 2>(sm, cb, lane);
        signal_count(sm, kDiagN, lane);
        if (kSolveFirst && has_next) producer_prefetch(p, ncs, nclen, h, hq, hk, pt, lo, f);
        const TileJob j1[2] = {{1, 1, 0}, {1, 2, 0}};
        run_tiles(sm, cb, j1, p.scale, lane);
        const TileJob j2[2] = {{2, 0, 0}, {2, 3, 3}};
        run_tiles(sm, cb, j2, p.scale, lane);
        break;
      }
      case 2: {
        diag_tiles<2, 3>(sm, cb, lane);
        signal_count(sm, kDiagN, lane);
        if (kSolveFirst && has_next) producer_prefetch(p, ncs, nclen, h, hq, hk, pt, lo, f);
        const TileJob j1[2] = {{1, 3, 0}, {1, 2, 1}};
        run_tiles(sm, cb, j1, p.scale, lane);
        const TileJob j2[2] = {{2, 1, 0}, {2, 3, 0}};
        run_tiles(sm, cb, j2, p.scale, lane);
        break;
      }
      default: {
        diag_tiles<3, 4>(sm, cb, lane);
        signal_count(sm, kDiagN, lane);
        if (kSolveFirst && has_next) producer_prefetch(p, ncs, nclen, h, hq, hk, pt, lo, f);
        const TileJob j1[2] = {{1, 3, 1}, {1, 3, 2}};
        run_tiles(sm, cb, j1, p.scale, lane);
        const TileJob j2[2] = {{2, 1, 1}, {2, 2, 0}};
        run_tiles(sm, cb, j2, p.scale, lane);
        break;
      }
    }
    signal_count(sm, kPPhase, lane);
    wait_count<V::kHooks>(sm, kPPhase, 4 * (2 * u + 2));  // diagonal blocks and N tiles done

    // 3: off-diagonal blocks of T~ (waves 1 and 3), the remaining P tiles (two
    // each on waves 0 and 2), V once the consumers have read the previous chunk's
    switch (pw) {
      case 0: {
        if (kSolveFirst && has_next) producer_prefetch(p, ncs, nclen, h, hq, hk, pt, lo, f);
        const TileJob j1[2] = {{2, 2, 1}, {2, 2, 2}};
        run_tiles(sm, cb, j1, p.scale, lane);
        if (has_next) gts = chunk_gates(f, lane, nclen, neg_decay, dt_bias);  // the next chunk's gates
        break;
      }
      case 1: {
        offdiag_right(sm, cb, u, lane);
        break;
      }
      case 2: {
        const TileJob j1[2] = {{2, 3, 1}, {2, 3, 2}};
        run_tiles(sm, cb, j1, p.scale, lane);
        break;
      }
      default:
        offdiag_left<V::kHooks>(sm, cb, u, lane);
        break;
    }
    if (u >= 1) wait_count<V::kHooks>(sm, kVFree, V::NCW * u);
#pragma unroll
    for (int it = 0; it < NVIT; ++it) {
      const int seg = pt + it * NPROD;
      if (seg < V::VSEG)
        *reinterpret_cast<uint4*>(sm.V + (seg / (V::ROWS / 8)) * VSTR + 8 * (seg % (V::ROWS / 8))) = fv[it];
    }
    __builtin_amdgcn_s_setprio(0);
    if (!V::kHooks || p.ready_chunks <= 0 || t < p.ready_chunks) signal_count(sm, kReady, lane);
  }
  if constexpr (!V::kPersist) {
    break;
  } else {
    k = next_chain(sm, k + 1);
    if (k >= chain_count(sm)) break;
    s0 = sm.ps0[k];
    s1 = sm.ps1[k];
    nchunks = int((s1 - s0 + C - 1) / C);
  }
  }
  if constexpr (V::kCopy) {
    wait_count<V::kHooks>(sm, kReady, 4 * nchunks);
    copy_tiles_out<Smem>(chunk_bufs(sm, (nchunks - 1) & 1), images + int64_t(nchunks - 1) * p.Hv * kTileImage, pt,
                   aborted(sm));
  }
}

// The raw gate inputs (a, b) of token `lane` of a chunk, clamped into the chunk.
template <int NT>
__device__ __forceinline__ void prefetch_gate_inputs(const PrefillArgs& p, int64_t cs, int clen, int h, int lane,
                                                     ProducerPrefetchT<NT>& f) {
  const int off = (lane < clen ? lane : clen - 1) * p.Hv;
  f.a = (p.a + cs * p.Hv + h)[off];
  f.b = (p.b + cs * p.Hv + h)[off];
}

template <int SI, class Smem>
__device__ __forceinline__ void diag_tile_of(Smem& sm, const ChunkBufs& cb, int lane) {
  diag_tiles<SI, SI + 1>(sm, cb, lane);
}

// The producer loop of split chains, pipelined one step deep: seven producer
// waves beside one consumer (chains split 8 ways) or six beside two (split 4
// ways), with NS = NP - 3 of them stagers.  For chunk t:
//   * wave 0 solves the diagonal blocks of T~ once chunk t's four diagonal N tiles
//     are in, then forms chunk t + 1's gates (and, with three stagers, chunk t + 1's
//     last diagonal N tile);
//   * waves 1 and 3 form the six off-diagonal N tiles (and one P tile each), then
//     the off-diagonal blocks of T~ (offdiag_right, offdiag_left);
//   * the stager waves (2, 4, 5[, 6]) form the other eight P tiles and stage V, then
//     stage chunk t + 1's K and Q and form its other diagonal N tiles,
// so the solve of chunk t + 1 can start as soon as chunk t's is done, instead of
// after chunk t + 1's staging and diagonal tiles.  Hand-offs per chunk: kStaged
// NS + 1 (the stagers' K/Q and wave 0's gates), kVStaged NS, kDiagN 4, kPPhase 3
// (the solve, and the N tiles of waves 1 and 3), kNRead 1 (the left off-diagonal
// wave read its N operands, so the next chunk's N tiles may overwrite them), kX32
// 1, kReady NS + 2 (waves 1 and 3, the stagers).  Every buffer of chunk t + 1's
// parity is written only after the consumers signalled chunk t - 1 consumed.
template <class V>
__device__ __forceinline__ void producer_loop_split(PrefillSmem& sm, const PrefillArgs& p, int64_t s0, int64_t s1,
                                                    int nchunks, int h, int hq, int hk, int row0, int pw,
                                                    int lane0) {
  static_assert(V::kPipelined && !V::kLoad && !V::kCopy, "pipelined producer loop of split chains");
  constexpr int NS = V::kStagers, NST = 64 * NS;        // stager waves, threads
  constexpr int NVIT = (V::VSEG + NST - 1) / NST;       // V segments per stager thread
  const int si = pw == 2 ? 0 : pw >= 4 ? pw - 3 : -1;   // stager index (waves 2, 4, 5, 6)
  const int pt = (si < 0 ? 0 : si) * 64 + lane0;        // thread index among the stagers
  const float neg_decay = -expf(p.A_log[h]);
  const float dt_bias = p.dt_bias[h];
  const LaneOffsets lo = {(pt >> 4) * p.Hk * D + 8 * (pt & 15), (pt >> 4) * p.Hq * D + 8 * (pt & 15), pt * p.Hv};
  int voff[NVIT], vrow[NVIT];
#pragma unroll
  for (int it = 0; it < NVIT; ++it) {
    const int seg = pt + it * NST, c = seg / (V::ROWS / 8), sg = seg % (V::ROWS / 8);
    vrow[it] = seg < V::VSEG ? c : C;  // C: no segment
    voff[it] = c * p.Hv * D + 8 * sg;
  }
  auto chunk_len = [&](int64_t cs) { return int(s1 - cs < C ? s1 - cs : C); };
  auto load_v = [&](uint4 (&fv)[NVIT], int64_t cs) {
    const uint16_t* vb = p.v + (cs * p.Hv + h) * D + row0;
    const int clen = chunk_len(cs);
#pragma unroll
    for (int it = 0; it < NVIT; ++it) {
      fv[it] = uint4{0u, 0u, 0u, 0u};
      if (vrow[it] < clen) fv[it] = *reinterpret_cast<const uint4*>(vb + voff[it]);
    }
  };
  // Diagonal N tiles: stager si forms tile si; with three stagers wave 0 forms tile 3.
  auto diag_tile = [&](const ChunkBufs& cb, int lane) {
    switch (si) {
      case 0: diag_tile_of<0>(sm, cb, lane); break;
      case 1: diag_tile_of<1>(sm, cb, lane); break;
      case 2: diag_tile_of<2>(sm, cb, lane); break;
      default: diag_tile_of<3>(sm, cb, lane); break;
    }
  };
  auto ready = [&](int t, int lane) {
    if (!V::kHooks || p.ready_chunks <= 0 || t < p.ready_chunks) signal_count(sm, kReady, lane);
  };
  // The stagers' eight P tiles (P(2,2) and P(3,3) go to waves 3 and 1).
  auto stager_tiles = [&](const ChunkBufs& cb, int lane) {
    if constexpr (NS == 4) {
      const TileJob jobs[4][2] = {{{2, 0, 0}, {2, 1, 0}}, {{2, 1, 1}, {2, 2, 0}}, {{2, 2, 1}, {2, 3, 0}},
                                  {{2, 3, 1}, {2, 3, 2}}};
      switch (si) {
        case 0: run_tiles(sm, cb, jobs[0], p.scale, lane); break;
        case 1: run_tiles(sm, cb, jobs[1], p.scale, lane); break;
        case 2: run_tiles(sm, cb, jobs[2], p.scale, lane); break;
        default: run_tiles(sm, cb, jobs[3], p.scale, lane); break;
      }
    } else {
      static_assert(NS == 3, "three or four stagers");
      const TileJob a0[2] = {{2, 0, 0}, {2, 1, 0}}, a1[1] = {{2, 1, 1}};
      const TileJob b0[2] = {{2, 2, 0}, {2, 2, 1}}, b1[1] = {{2, 3, 0}};
      const TileJob c0[2] = {{2, 3, 1}, {2, 3, 2}};
      switch (si) {
        case 0: run_tiles(sm, cb, a0, p.scale, lane); run_tiles(sm, cb, a1, p.scale, lane); break;
        case 1: run_tiles(sm, cb, b0, p.scale, lane); run_tiles(sm, cb, b1, p.scale, lane); break;
        default: run_tiles(sm, cb, c0, p.scale, lane); break;
      }
    }
  };

  ProducerPrefetchT<NST> f = {};
  uint4 fv[NVIT];
  // Chunk 0 ahead of the loop: its gates, K/Q, and diagonal N tiles.
  if (pw == 0) {
    prefetch_gate_inputs(p, s0, chunk_len(s0), h, lane0, f);
    store_gates(chunk_bufs(sm, 0), chunk_gates(f, lane0, chunk_len(s0), neg_decay, dt_bias), lane0);
    signal_count(sm, kStaged, lane0);
    if (nchunks > 1) prefetch_gate_inputs(p, s0 + C, chunk_len(s0 + C), h, lane0, f);
    if constexpr (NS == 3) {
      wait_count<V::kHooks>(sm, kStaged, NS + 1);
      diag_tile_of<3>(sm, chunk_bufs(sm, 0), lane0);
      signal_count(sm, kDiagN, lane0);
    }
  } else if (si >= 0) {
    producer_prefetch(p, s0, chunk_len(s0), h, hq, hk, pt, lo, f);
    load_v(fv, s0);
    stage_kq(chunk_bufs(sm, 0), f, pt);
    signal_count(sm, kStaged, lane0);
    if (nchunks > 1) producer_prefetch(p, s0 + C, chunk_len(s0 + C), h, hq, hk, pt, lo, f);
    wait_count<V::kHooks>(sm, kStaged, NS + 1);
    diag_tile(chunk_bufs(sm, 0), lane0);
    signal_count(sm, kDiagN, lane0);
  }

  for (int t = 0; t < nchunks; ++t) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int64_t cs = s0 + int64_t(t) * C;
    const int64_t ncs = cs + C;
    const ChunkBufs cb = chunk_bufs(sm, t & 1);
    __builtin_amdgcn_s_setprio(1);
    switch (pw) {
      case 0:
        wait_count<V::kHooks>(sm, kDiagN, 4 * (t + 1));
        diag_solve(sm, cb, lane);
        signal_count(sm, kPPhase, lane);
        if (ncs < s1) {
          // Chunk t + 1's gates, stored into the buffers of chunk t - 1 once consumed.
          const ChunkGates g = chunk_gates(f, lane, chunk_len(ncs), neg_decay, dt_bias);
          if (t >= 1) wait_count<V::kHooks>(sm, kConsumed, V::NCW * t);
          const ChunkBufs cbn = chunk_bufs(sm, (t + 1) & 1);
          store_gates(cbn, g, lane);
          signal_count(sm, kStaged, lane);
          if (ncs + C < s1) prefetch_gate_inputs(p, ncs + C, chunk_len(ncs + C), h, lane, f);
          if constexpr (NS == 3) {
            // Chunk t + 1's last diagonal N tile, once its K is staged (the solve of
            // chunk t, just done, freed the scratch).
            wait_count<V::kHooks>(sm, kStaged, (NS + 1) * (t + 2));
            diag_tile_of<3>(sm, cbn, lane);
            signal_count(sm, kDiagN, lane);
          }
        }
        break;
      case 1: {
        wait_count<V::kHooks>(sm, kStaged, (NS + 1) * (t + 1));
        if (t >= 1) wait_count<V::kHooks>(sm, kNRead, t);  // chunk t - 1's N read by the left wave
        const TileJob j1[2] = {{1, 2, 1}, {1, 3, 2}};
        run_tiles(sm, cb, j1, p.scale, lane);
        const TileJob j2[2] = {{1, 3, 1}, {2, 3, 3}};
        run_tiles(sm, cb, j2, p.scale, lane);
        signal_count(sm, kPPhase, lane);
        wait_count<V::kHooks>(sm, kPPhase, 3 * (t + 1));
        offdiag_right(sm, cb, t, lane);
        ready(t, lane);
        break;
      }
      case 3: {
        wait_count<V::kHooks>(sm, kStaged, (NS + 1) * (t + 1));
        const TileJob j1[2] = {{1, 1, 0}, {1, 2, 0}};
        run_tiles(sm, cb, j1, p.scale, lane);
        const TileJob j2[2] = {{1, 3, 0}, {2, 2, 2}};
        run_tiles(sm, cb, j2, p.scale, lane);
        signal_count(sm, kPPhase, lane);
        wait_count<V::kHooks>(sm, kPPhase, 3 * (t + 1));
        offdiag_left<V::kHooks, true>(sm, cb, t, lane);
        ready(t, lane);
        break;
      }
      default: {  // stagers
        // Chunk t's V as soon as the consumers have read chunk t - 1's: with K, Q and
        // the gates (staged a tick ahead) it is all their retrieve and Y need.
        if (t >= 1) wait_count<V::kHooks>(sm, kVFree, V::NCW * t);
#pragma unroll
        for (int it = 0; it < NVIT; ++it) {
          const int seg = pt + it * NST;
          if (seg < V::VSEG)
            *reinterpret_cast<uint4*>(sm.V + (seg / (V::ROWS / 8)) * VSTR + 8 * (seg % (V::ROWS / 8))) = fv[it];
        }
        signal_count(sm, kVStaged, lane);
        if (ncs < s1) load_v(fv, ncs);  // chunk t + 1's V into registers
        wait_count<V::kHooks>(sm, kStaged, (NS + 1) * (t + 1));  // chunk t's gates (wave 0)
        stager_tiles(cb, lane);
        ready(t, lane);  // chunk t's P tiles
        if (ncs < s1) {
          // Chunk t + 1: K and Q into the buffers of chunk t - 1 once consumed; its
          // diagonal N tiles once the solve of chunk t freed their scratch.
          if (t >= 1) wait_count<V::kHooks>(sm, kConsumed, V::NCW * t);
          const ChunkBufs cbn = chunk_bufs(sm, (t + 1) & 1);
          stage_kq(cbn, f, pt);
          signal_count(sm, kStaged, lane);
          if (ncs + C < s1) producer_prefetch(p, ncs + C, chunk_len(ncs + C), h, hq, hk, pt, lo, f);
          wait_count<V::kHooks>(sm, kStaged, (NS + 1) * (t + 2));
          wait_count<V::kHooks>(sm, kPPhase, 3 * (t + 1));
          diag_tile(cbn, lane);
          signal_count(sm, kDiagN, lane);
        }
        break;
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }
}

// The loader loop of the two-kernel path: the producers' hand-offs and staging,
// with chunk t's T~ (hi, lo), P and gates copied from their prepared images (tiles
// = image of chunk 0 of this chain; chunk t is Hv images further) instead of
// computed.  K and Q are staged as the producers stage them, V at the end of the
// tick, after the consumers' last read of the previous chunk's V.
// The images of chunk t + 1 are loaded into registers during tick t, so their
// latency overlaps the waits for the consumers; with V::kDeepImages the images of
// chunk t + 2 (two register sets, alternating), as soon as chunk t's are in LDS.
// V goes two chunks ahead in every variant (two register sets): the prep kernel does
// not read V, so with inputs that the caches do not hold its loads come from HBM
// (config 3 with four rotating input sets: 142.5 -> 132.0 us, unchanged with one).
template <class V>
__device__ __forceinline__ void loader_loop(PrefillSmem& sm, const PrefillArgs& p, const u32x4* tiles, int64_t s0,
                                            int64_t s1, int nchunks, int h, int hq, int hk, int row0, int pw,
                                            int lane0) {
  constexpr int NVIT = (V::VSEG + NPROD - 1) / NPROD;        // V segments per loader thread
  constexpr int NTIT = (kTileImage + NPROD - 1) / NPROD;     // 16-byte tile units per loader thread
  constexpr int NT1 = kTileUnits1;                           // 16-byte units per tile image
  const int pt = pw * 64 + lane0;
  const LaneOffsets lo = {(pt >> 4) * p.Hk * D + 8 * (pt & 15), (pt >> 4) * p.Hq * D + 8 * (pt & 15), pt * p.Hv};
  int voff[NVIT], vrow[NVIT];
#pragma unroll
  for (int it = 0; it < NVIT; ++it) {
    const int seg = pt + it * NPROD, c = seg / (V::ROWS / 8), sg = seg % (V::ROWS / 8);
    vrow[it] = seg < V::VSEG ? c : C;  // C: no segment
    voff[it] = c * p.Hv * D + 8 * sg;
  }
  // Unit pt + 256 it of a chunk's images (the last round's excess lanes re-read
  // the last unit and store nothing).
  int toff[NTIT];
#pragma unroll
  for (int it = 0; it < NTIT; ++it) toff[it] = pt + it * NPROD < kTileImage ? pt + it * NPROD : kTileImage - 1;
  // (First-class vectors: copies of uint4 structs would go through the stack.)
  constexpr bool deep = V::kDeepImages;
  u32x4 tva[NTIT], tvb[deep ? NTIT : 1], fva[NVIT], fvb[NVIT];
  // V slice of chunk t (tokens [s0 + C t, s1) of it) into fv, zero past the sequence.
  auto load_v = [&](int t, u32x4(&fv)[NVIT]) {
    const int64_t vs = s0 + int64_t(t) * C;
    const int vlen = int(s1 - vs < C ? s1 - vs : C);
    const uint16_t* vb = p.v + (vs * p.Hv + h) * D + row0;
#pragma unroll
    for (int it = 0; it < NVIT; ++it) {
      fv[it] = u32x4{0u, 0u, 0u, 0u};
      if (vrow[it] < vlen) fv[it] = *reinterpret_cast<const u32x4*>(vb + voff[it]);
    }
  };
  ProducerPrefetch f;
  producer_prefetch(p, s0, int(s1 - s0 < C ? s1 - s0 : C), h, hq, hk, pt, lo, f);
  // Chunk 0's images (and chunk 1's), and the V slices of chunks 0 and 1, into registers.
#pragma unroll
  for (int it = 0; it < NTIT; ++it) tva[it] = tiles[toff[it]];
  if constexpr (deep) {
    if (nchunks > 1) {
      const u32x4* src = tiles + int64_t(p.Hv) * kTileImage;
#pragma unroll
      for (int it = 0; it < NTIT; ++it) tvb[it] = src[toff[it]];
    }
  }
  load_v(0, fva);
  if (nchunks > 1) load_v(1, fvb);

  // Tick t stages chunk t from the register sets tv (images) and fv (V), then loads
  // chunk t + 2's V into fv (the V loads go two chunks ahead, so that their latency
  // from HBM, when the inputs are not in the caches, stays off the chain).
  auto tick = [&](int t, u32x4(&tv)[NTIT], u32x4(&fv)[NVIT]) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int64_t cs = s0 + int64_t(t) * C;
    const int64_t ncs = cs + C;
    const int nclen = int(s1 - ncs < C ? s1 - ncs : C);
    const ChunkBufs cb = chunk_bufs(sm, t & 1);
    if (t >= 2) wait_count<V::kHooks>(sm, kConsumed, V::NCW * (t - 1));  // chunk t - 2 consumed
    stage_kq(cb, f, pt);
#pragma unroll
    for (int it = 0; it < NTIT; ++it) {
      const int e = pt + it * NPROD;
      if (e < kTileUnits) {
        uint16_t* dst = e < NT1       ? cb.Th + tile_unit_off(e)
                        : e < 2 * NT1 ? cb.Tl + tile_unit_off(e - NT1)
                                      : cb.P + tile_unit_off(e - 2 * NT1);
        *reinterpret_cast<u32x4*>(dst) = tv[it];
      } else if (e < kTileImage) {
        *reinterpret_cast<u32x4*>(gate_unit<PrefillSmem>(cb, e - kTileUnits)) = tv[it];
      }
    }
    if (t >= 1) wait_count<V::kHooks>(sm, kVFree, V::NCW * t);  // the consumers' last read of V
#pragma unroll
    for (int it = 0; it < NVIT; ++it) {
      const int seg = pt + it * NPROD;
      if (seg < V::VSEG)
        *reinterpret_cast<u32x4*>(sm.V + (seg / (V::ROWS / 8)) * VSTR + 8 * (seg % (V::ROWS / 8))) = fv[it];
    }
    signal_count(sm, kReady, lane);
    // The next chunks' loads go out after the hand-off.  Issued before it, the
    // waits for this tick's registers (loaded a tick earlier) would also wait for
    // them: the K/Q loads are conditional, so the compiler cannot count them and
    // waits for every load issued since.
    if (ncs < s1) producer_prefetch(p, ncs, nclen, h, hq, hk, pt, lo, f);
    if (deep && t + 2 < nchunks) {  // chunk t + 2's images into this set
      const u32x4* src = tiles + int64_t(t + 2) * p.Hv * kTileImage;
#pragma unroll
      for (int it = 0; it < NTIT; ++it) tv[it] = src[toff[it]];
    }
    if (!deep && t + 1 < nchunks) {  // chunk t + 1's images into registers
      const u32x4* src = tiles + int64_t(t + 1) * p.Hv * kTileImage;
#pragma unroll
      for (int it = 0; it < NTIT; ++it) tv[it] = src[toff[it]];
    }
    if (t + 2 < nchunks) load_v(t + 2, fv);  // chunk t + 2's V slice
  };
  for (int t = 0; t < nchunks; t += 2) {
    tick(t, tva, fva);
    if (t + 1 < nchunks) {
      if constexpr (deep) {
        tick(t + 1, tvb, fvb);
      } else {
        tick(t + 1, tva, fvb);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Consumer side (waves 0 .. NCW-1; wave w owns state rows R0 + VW w .. + VW - 1)
// ---------------------------------------------------------------------------

// Xk = K S^T (rows c, cols v) with S as hi/lo B operands, and Xq = (Q S^T)^T
// (rows v, cols c) with S's hi part as the A operand (output-only product).
template <int VT>
__device__ __forceinline__ void retrieve(const ChunkBufs& cb, const f32x4 (&S)[VT][8], f32x4 (&Xk)[4][VT],
                                         f32x4 (&Xq)[VT][4], int lane) {
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) Xk[ct][vt] = Xq[vt][ct] = zero4();
  if constexpr (VT == 1) {
    // One state tile leaves registers for the next contraction block's K and Q
    // fragments: they are read while this block's MFMAs run (the scheduling
    // barrier keeps the reads ahead of them).
    uint4 kf[2][4], qf[2][4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      kf[0][ct] = frag_kq(cb.K, 16 * ct, 0, lane);
      qf[0][ct] = frag_kq(cb.Q, 16 * ct, 0, lane);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks < 3) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          kf[(ks + 1) & 1][ct] = frag_kq(cb.K, 16 * ct, ks + 1, lane);
          qf[(ks + 1) & 1][ct] = frag_kq(cb.Q, 16 * ct, ks + 1, lane);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      uint4 Sh, Sl;
      split_pack(S[0][2 * ks], S[0][2 * ks + 1], Sh, Sl);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        Xk[ct][0] = mfma(kf[ks & 1][ct], Sh, Xk[ct][0]);
        Xk[ct][0] = mfma(kf[ks & 1][ct], Sl, Xk[ct][0]);
        Xq[0][ct] = mfma(Sh, qf[ks & 1][ct], Xq[0][ct]);
      }
    }
    return;
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 Sh[VT], Sl[VT];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) split_pack(S[vt][2 * ks], S[vt][2 * ks + 1], Sh[vt], Sl[vt]);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const uint4 ak = frag_kq(cb.K, 16 * ct, ks, lane);
      const uint4 bq = frag_kq(cb.Q, 16 * ct, ks, lane);
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        Xk[ct][vt] = mfma(ak, Sh[vt], Xk[ct][vt]);
        Xk[ct][vt] = mfma(ak, Sl[vt], Xk[ct][vt]);
        Xq[vt][ct] = mfma(Sh[vt], bq, Xq[vt][ct]);
      }
    }
  }
}

// State row (within the wave's VW rows) held by column n of state tile vt.  With two
// tiles the rows interleave in groups of four (tile 0: 0-3, 8-11, ..., tile 1: 4-7,
// 12-15, ...), so that a lane's output rows of the two tiles are 8 consecutive values.
template <int VT>
__device__ __forceinline__ int vrow(int vt, int n) {
  return VT == 2 ? 8 * (n >> 2) + 4 * vt + (n & 3) : 16 * vt + n;
}

// The consumer loop: iteration t (>= 1) advances the state through chunk t-1
// from the buffers of parity (t-1) & 1, once the producers have handed it over.
// Column n of state tile vt is state row row0 + VW wave + vrow(vt, n) (V column
// VW wave + vrow(vt, n) of the staged slice).
template <class V>
__device__ __forceinline__ void consumer_loop(PrefillSmem& sm, const PrefillArgs& p, int64_t s0, int64_t s1,
                                              int nchunks, int h, int row0, int wave, int lane0,
                                              f32x4 (&S)[V::VT][8], int u0 = 0) {
  constexpr int VT = V::VT, VW = V::VW;
  const int64_t vstride = int64_t(p.Hv) * D;
  // Element offset of output row 16ct + lane%16, first column of the lane's output
  // values (8 (lane/16) with two state tiles, 4 (lane/16) with one), from the wave's
  // (uniform) chunk base.
  int orow[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) orow[ct] = (16 * ct + (lane0 & 15)) * int(vstride) + (VT == 2 ? 8 : 4) * (lane0 >> 4);
  for (int t = 1; t <= nchunks; ++t) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int g = lane >> 4, n16 = lane & 15;
    const int64_t cs = s0 + int64_t(t - 1) * C;
    const int clen = int(s1 - cs < C ? s1 - cs : C);
    // u: the chunk's position in the workgroup's stream of chunks (persistent
    // kernel: u0 chunks of earlier chains precede this chain's).
    const int u = u0 + t;
    const ChunkBufs cb = chunk_bufs(sm, (u - 1) & 1);
    if constexpr (V::kPipelined) {
      // Pipelined producers hand a chunk over in two steps: K, Q, the gates and V for
      // the retrieve and Y, then T~ and P ("ready", below) for v_new and the output.
      wait_count<V::kHooks>(sm, kStaged, (V::kStagers + 1) * u);
      wait_count<V::kHooks>(sm, kVStaged, V::kStagers * u);
    } else {
      wait_count<V::kHooks>(sm, kReady, 4 * u);  // chunk u - 1 prepared
    }

    // 1: X = K S^T, (Q S^T)^T
    f32x4 Xk[4][VT], Xq[VT][4];
    retrieve(cb, S, Xk, Xq, lane);

    // 2: Y, v_new, output
    // Y = beta (V - e^gamma X); element (c = 16ct + 4g + i, v = VW w + vrow(vt, n16)).
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const float4 bc = *reinterpret_cast<const float4*>(cb.bet + 16 * ct + 4 * g);
      const float4 ec = *reinterpret_cast<const float4*>(cb.eg + 16 * ct + 4 * g);
      const float b4[4] = {bc.x, bc.y, bc.z, bc.w}, e4[4] = {ec.x, ec.y, ec.z, ec.w};
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        // V rows 16ct + 4g .. +3 of column VW w + vrow(vt, n16): lane j of a 16-lane
        // group reads the 4 columns VW w + vrow(vt, 4 (j & 3)) .. +3 of row 16ct + 4g + j/4.
        const uint2 vv = read_tr(sm.V + (16 * ct + 4 * g + (n16 >> 2)) * VSTR + VW * wave + vrow<VT>(vt, 4 * (n16 & 3)));
        const float vf[4] = {bf16lo_f32(vv.x), bf16hi_f32(vv.x), bf16lo_f32(vv.y), bf16hi_f32(vv.y)};
#pragma unroll
        for (int i = 0; i < 4; ++i) Xk[ct][vt][i] = b4[i] * (vf[i] - e4[i] * Xk[ct][vt][i]);
      }
      const float ecn = cb.eg[16 * ct + n16] * p.scale;  // scale e^gamma of output column c = 16ct + n16
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) Xq[vt][ct] = Xq[vt][ct] * ecn;
    }
    signal_count(sm, kVFree, lane);  // V of this chunk read
    if constexpr (V::kPipelined) wait_count<V::kHooks>(sm, kReady, (V::kStagers + 2) * u);  // T~ and P
    // The 16-row consumer reads all its T~ and P operands now (they are ready), so that
    // their latency overlaps the Y split; the 32-row one, short of registers, as used.
    // Pair (ct, js) of T~ is fragment ct < 2 ? ct : 2 ct - 2 + js; pair (js, ct) of
    // P is fragment js ? ct + 2 : ct.
    constexpr int NPF = VT == 1 ? 6 : 1;
    uint4 thf[NPF], tlf[NPF], pqf[NPF];
    if constexpr (VT == 1) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int js = 0; js <= (ct >> 1); ++js) {
          const int i = ct < 2 ? ct : 2 * ct - 2 + js;
          thf[i] = frag(cb.Th, TSTR, 16 * ct, js, lane);
          tlf[i] = frag(cb.Tl, TSTR, 16 * ct, js, lane);
        }
#pragma unroll
      for (int js = 0; js < 2; ++js)
#pragma unroll
        for (int ct = 2 * js; ct < 4; ++ct) pqf[js ? ct + 2 : ct] = frag(cb.P, TSTR, 16 * ct, js, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
    // v_new = T~ Y (contraction over the rows of Y in blocks js; T~ is lower triangular).
    uint4 Yh[VT][2], Yl[VT][2];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int js = 0; js < 2; ++js) split_pack(Xk[2 * js][vt], Xk[2 * js + 1][vt], Yh[vt][js], Yl[vt][js]);
    f32x4 Vn[4][VT];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) Vn[ct][vt] = zero4();
#pragma unroll
      for (int js = 0; js <= (ct >> 1); ++js) {
        uint4 th, tl;
        if constexpr (VT == 1) {
          th = thf[ct < 2 ? ct : 2 * ct - 2 + js];
          tl = tlf[ct < 2 ? ct : 2 * ct - 2 + js];
        } else {
          th = frag(cb.Th, TSTR, 16 * ct, js, lane);
          tl = frag(cb.Tl, TSTR, 16 * ct, js, lane);
        }
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) {
          Vn[ct][vt] = mfma(th, Yh[vt][js], Vn[ct][vt]);
          Vn[ct][vt] = mfma(th, Yl[vt][js], Vn[ct][vt]);
          Vn[ct][vt] = mfma(tl, Yh[vt][js], Vn[ct][vt]);
        }
      }
    }
    // o^T = scale e^gamma (S Q^T) + v_new^T (scale P)^T (rows v, cols c); P is lower triangular.
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      uint4 vb[VT];
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) vb[vt] = pack_hi(Vn[2 * js][vt], Vn[2 * js + 1][vt]);
#pragma unroll
      for (int ct = 2 * js; ct < 4; ++ct) {
        uint4 pq;
        if constexpr (VT == 1) {
          pq = pqf[js ? ct + 2 : ct];
        } else {
          pq = frag(cb.P, TSTR, 16 * ct, js, lane);
        }
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) Xq[vt][ct] = mfma(vb[vt], pq, Xq[vt][ct]);
      }
    }
    // 3: S = e^{gamma_last} S + sum_c K[c]^T (d_c v_new[c]),  d_c = e^{gamma_last - gamma_c}
    const float dlast = cb.eg[clen - 1];
    uint4 Uh[VT][2], Ul[VT][2];
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      const float4 d0 = *reinterpret_cast<const float4*>(cb.dd + 32 * js + 4 * g);
      const float4 d1 = *reinterpret_cast<const float4*>(cb.dd + 32 * js + 16 + 4 * g);
      const f32x4 e0 = {d0.x, d0.y, d0.z, d0.w}, e1 = {d1.x, d1.y, d1.z, d1.w};
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) split_pack(Vn[2 * js][vt] * e0, Vn[2 * js + 1][vt] * e1, Uh[vt][js], Ul[vt][js]);
    }
    const KtBases kb = kt_bases(lane);
    static_for<8>([&](auto KT) {
      constexpr int kt = decltype(KT)::value;
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) S[vt][kt] = S[vt][kt] * dlast;
      static_for<2>([&](auto JS) {
        constexpr int js = decltype(JS)::value;
        const uint4 ak = frag_tr_k_at<js, kt>(cb.K, kb);
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) {
          S[vt][kt] = mfma(ak, Uh[vt][js], S[vt][kt]);
          S[vt][kt] = mfma(ak, Ul[vt][js], S[vt][kt]);
        }
      });
    });
    // The output stores, in the same block as the state update so that their packing
    // and issue fill the update's MFMA shadow.  Lane holds o[c = 16ct + n16][v = row0 +
    // VW w + vrow(vt, 4g + i)]: with two tiles 8 consecutive v (one 16-byte store per
    // ct), with one 4 (8 bytes).  Rows at or past clen fall outside the buffer
    // resource, whose extent ends at the chunk's last token: the hardware drops their
    // stores, so no lane needs a branch.
    {
      const BufferRsrc orsrc = buffer_rsrc(p.out + cs * vstride + (int64_t(h) * D + row0 + VW * wave),
                                           uint32_t(clen) * uint32_t(vstride) * 2u);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        if constexpr (VT == 2) {
          const f32x4 &o0 = Xq[0][ct], &o1 = Xq[1][ct];
          buffer_store16(u32x4{pack_bf16x2(o0[0], o0[1]), pack_bf16x2(o0[2], o0[3]), pack_bf16x2(o1[0], o1[1]),
                               pack_bf16x2(o1[2], o1[3])},
                         orsrc, 2 * orow[ct]);
        } else {
          const f32x4& o = Xq[0][ct];
          buffer_store8(u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])}, orsrc, 2 * orow[ct]);
        }
      }
    }
    signal_count(sm, kConsumed, lane);  // buffers of this chunk no longer read
  }
}

// The token-split consumer loop of the two-kernel state pass (F = 8).  The four
// consumer waves share the slice's 16 state rows: wave w keeps state columns
// 32w .. 32w + 31 in fp32, forms the rows of X = K S^T, Y and the output of the
// chunk's tokens 16w .. 16w + 15, and updates its own columns.  Two LDS exchanges a
// chunk give every wave what the others formed: the four blocks of Y (for v_new, which
// every wave forms whole) and the bf16 hi/lo parts of the four column blocks of the
// state (for the next retrieve).  Each value is produced by the same operations in the
// same order as in consumer_loop with one 16-row wave, so the results are
// bit-identical, while the chain of a chunk loses three quarters of the retrieve, Y,
// the output and the state update.
//
// Each exchange buffer is single: a wave rewrites its block of Y (of the state) only
// after the wait for all four blocks of the other exchange, which every wave signals
// after its last read of the previous contents.
template <class V>
__device__ __forceinline__ void consumer_loop_tsplit(PrefillSmem& sm, const PrefillArgs& p, int64_t s0, int64_t s1,
                                                     int nchunks, int h, int row0, int wave, int lane0,
                                                     f32x4 (&S)[2]) {
  static_assert(V::kTokenSplit && V::VT == 1 && V::NCW == 4, "token-split consumers");
  const int64_t vstride = int64_t(p.Hv) * D;
  const int ct = wave;  // this wave's 16-token block and 32-column block
  const int orow = (16 * ct + (lane0 & 15)) * int(vstride) + 4 * (lane0 >> 4);
  f32x4* const yx = reinterpret_cast<f32x4*>(sm.Nh);            // Y: [block][lane]
  uint4* const sx = reinterpret_cast<uint4*>(sm.Nh) + 4 * 64;   // state: [block][hi, lo][lane]
  // K^T operand base of column blocks 2 ct, 2 ct + 1 (kt_bases with kt / 2 = ct).
  int ktb;
  {
    const int j = lane0 & 15, rl = 4 * (lane0 >> 4) + (j >> 2), sl = kq_sigma(rl);
    ktb = rl * KSTR + 8 * ((j & 3) ^ (sl & 3)) + 32 * (ct ^ (sl >> 2));
  }
  {
    uint4 Sh, Sl;
    split_pack(S[0], S[1], Sh, Sl);
    sx[(2 * ct) * 64 + lane0] = Sh;
    sx[(2 * ct + 1) * 64 + lane0] = Sl;
    signal_count(sm, kSx, lane0);
  }
  for (int t = 1; t <= nchunks; ++t) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int g = lane >> 4, n16 = lane & 15;
    const int64_t cs = s0 + int64_t(t - 1) * C;
    const int clen = int(s1 - cs < C ? s1 - cs : C);
    const ChunkBufs cb = chunk_bufs(sm, (t - 1) & 1);
    // Chunk t - 1 loaded; the state after chunk t - 2 looked at in the same read.
    const bool sx_ready = wait_count_peek<V::kHooks>(sm, kReady, 4 * t, kSx, 4 * t);
    uint4 kf[4], qf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kf[ks] = frag_kq(cb.K, 16 * ct, ks, lane);
      qf[ks] = frag_kq(cb.Q, 16 * ct, ks, lane);
    }
    if (!sx_ready) wait_count<V::kHooks>(sm, kSx, 4 * t);  // the state after chunk t - 2
    uint4 Sh[4], Sl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      Sh[ks] = sx[(2 * ks) * 64 + lane];
      Sl[ks] = sx[(2 * ks + 1) * 64 + lane];
    }

    // 1: block ct of X = K S^T and of (Q S^T)^T.
    f32x4 xk = zero4(), xq = zero4();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      xk = mfma(kf[ks], Sh[ks], xk);
      xk = mfma(kf[ks], Sl[ks], xk);
      xq = mfma(Sh[ks], qf[ks], xq);
    }

    // 2: Y for rows c = 16ct + 4g + i, as consumer_loop; the output block scaled.
    {
      const float4 bc = *reinterpret_cast<const float4*>(cb.bet + 16 * ct + 4 * g);
      const float4 ec = *reinterpret_cast<const float4*>(cb.eg + 16 * ct + 4 * g);
      const float b4[4] = {bc.x, bc.y, bc.z, bc.w}, e4[4] = {ec.x, ec.y, ec.z, ec.w};
      const uint2 vv = read_tr(sm.V + (16 * ct + 4 * g + (n16 >> 2)) * VSTR + vrow<1>(0, 4 * (n16 & 3)));
      const float vf[4] = {bf16lo_f32(vv.x), bf16hi_f32(vv.x), bf16lo_f32(vv.y), bf16hi_f32(vv.y)};
#pragma unroll
      for (int i = 0; i < 4; ++i) xk[i] = b4[i] * (vf[i] - e4[i] * xk[i]);
      xq = xq * (cb.eg[16 * ct + n16] * p.scale);
    }
    signal_count(sm, kVFree, lane);  // V of this chunk read
    yx[64 * ct + lane] = xk;
    signal_count(sm, kYx, lane);
    // T~ (all of it) and this block's P operands, read while the other blocks arrive.
    uint4 thf[6], tlf[6];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int js = 0; js <= (c >> 1); ++js) {
        const int i = c < 2 ? c : 2 * c - 2 + js;
        thf[i] = frag(cb.Th, TSTR, 16 * c, js, lane);
        tlf[i] = frag(cb.Tl, TSTR, 16 * c, js, lane);
      }
    const uint4 pq0 = frag(cb.P, TSTR, 16 * ct, 0, lane);
    const uint4 pq1 = frag(cb.P, TSTR, 16 * ct, 1, lane);
    wait_count<V::kHooks>(sm, kYx, 4 * t);
    f32x4 Y[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) Y[c] = yx[64 * c + lane];

    // v_new = T~ Y, all 64 rows.
    uint4 Yh[2], Yl[2];
#pragma unroll
    for (int js = 0; js < 2; ++js) split_pack(Y[2 * js], Y[2 * js + 1], Yh[js], Yl[js]);
    f32x4 Vn[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      Vn[c] = zero4();
#pragma unroll
      for (int js = 0; js <= (c >> 1); ++js) {
        const uint4 th = thf[c < 2 ? c : 2 * c - 2 + js], tl = tlf[c < 2 ? c : 2 * c - 2 + js];
        Vn[c] = mfma(th, Yh[js], Vn[c]);
        Vn[c] = mfma(th, Yl[js], Vn[c]);
        Vn[c] = mfma(tl, Yh[js], Vn[c]);
      }
    }

    // 3: columns 32ct .. 32ct + 31 of S = e^{gamma_last} S + sum_c K[c]^T (d_c v_new[c]).
    const float dlast = cb.eg[clen - 1];
    uint4 Uh[2], Ul[2];
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      const float4 d0 = *reinterpret_cast<const float4*>(cb.dd + 32 * js + 4 * g);
      const float4 d1 = *reinterpret_cast<const float4*>(cb.dd + 32 * js + 16 + 4 * g);
      const f32x4 e0 = {d0.x, d0.y, d0.z, d0.w}, e1 = {d1.x, d1.y, d1.z, d1.w};
      split_pack(Vn[2 * js] * e0, Vn[2 * js + 1] * e1, Uh[js], Ul[js]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      S[j] = S[j] * dlast;
#pragma unroll
      for (int js = 0; js < 2; ++js) {
        const uint16_t* kp = cb.K + ktb + 32 * js * KSTR + 4 * j;
        const uint2 a = read_tr(kp), b = read_tr(kp + 16 * KSTR);
        const uint4 ak = uint4{a.x, a.y, b.x, b.y};
        S[j] = mfma(ak, Uh[js], S[j]);
        S[j] = mfma(ak, Ul[js], S[j]);
      }
    }
    signal_count(sm, kConsumed, lane);  // buffers of this chunk no longer read
    {
      uint4 h2, l2;
      split_pack(S[0], S[1], h2, l2);
      sx[(2 * ct) * 64 + lane] = h2;
      sx[(2 * ct + 1) * 64 + lane] = l2;
      signal_count(sm, kSx, lane);
    }

    // Output block ct: o^T = scale e^gamma (S Q^T) + v_new^T (scale P)^T.
    xq = mfma(pack_hi(Vn[0], Vn[1]), pq0, xq);
    if (ct >= 2) xq = mfma(pack_hi(Vn[2], Vn[3]), pq1, xq);
    // Rows at or past clen fall outside the buffer resource, whose extent ends at the
    // chunk's last token: the hardware drops their stores (no per-lane branch).
    {
      const BufferRsrc orsrc =
          buffer_rsrc(p.out + cs * vstride + (int64_t(h) * D + row0), uint32_t(clen) * uint32_t(vstride) * 2u);
      buffer_store8(u32x2{pack_bf16x2(xq[0], xq[1]), pack_bf16x2(xq[2], xq[3])}, orsrc, 2 * orow);
    }
  }
}

// The sequence of rank `rank` in descending length order (ties: lower index
// first), so the longest chains start first; natural order for large batches.
template <int NTHREADS>
__device__ int pick_sequence(PrefillSmem& sm, const PrefillArgs& p, int rank, int tid) {
  if (p.N <= 1 || p.N > kMaxSortedSeqs) return rank;
  int* len = reinterpret_cast<int*>(sm.Nh);  // scratch until the first chunk
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

// Workgroup b handles slice f of chain `chain` (chain = rank-major, v-head
// minor).  With F > 1 the F slices of chain c are b = 16 F (c / 16) + 8 (F (c % 2)
// + f) + (c % 16) / 2: workgroups are dealt to the XCDs round-robin, so the slices
// of one chain, and those of its GQA partner (chain c ^ 1), share an XCD (and its
// L2) for their common K/Q reads.  With F == 1 the two chains of a GQA pair share an
// XCD the same way.
template <class V>
__global__ __launch_bounds__(V::NTHREADS) void gdn_prefill_kernel(PrefillArgs p) {
  constexpr int NCW = V::NCW, VT = V::VT, VW = V::VW, NTHREADS = V::NTHREADS;
  __shared__ PrefillSmem sm;

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int hw = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Role index.  Waves are dealt to the four SIMDs round-robin.  In the loader
  // variant with one consumer, the consumer takes hardware wave 3, a SIMD to itself,
  // and two (mostly idle) loaders share SIMD 0: config 3 174 -> 170 us.  Elsewhere
  // the natural order measured as fast or faster (two consumers on SIMDs of their
  // own: +1.5%; the producer variant's solve wave sharing a SIMD: +7%).
  // With seven producers (beside one consumer) the consumer keeps hardware wave 0 and
  // shares its SIMD with the producer that has least to do (wave 0, the solve): hardware
  // waves 1-7 take producers 1, 2, 3, 0, 4, 5, 6.  With six (beside two consumers on
  // hardware waves 0 and 1) hardware waves 2-7 take producers 2, 3, 0, 5, 1, 4: the
  // consumers share their SIMDs with the solve wave and the third stager, and each
  // off-diagonal wave shares one with a stager (1.5-2.5% faster than pairing the
  // second consumer with the right off-diagonal wave, or the two off-diagonal waves).
  const int wave = V::NP == 7   ? (hw == 0 ? 0 : 1 + ((0x6540321 >> (4 * (hw - 1))) & 15))
                   : V::NP == 6 ? (hw < 2 ? hw : 2 + ((0x415032 >> (4 * (hw - 2))) & 15))
                   : !(V::kLoad && NCW == 1) ? hw
                   : hw == 3 ? 0 : hw < 3 ? hw + 1 : hw;

  const int bid = blockIdx.x;
  // Workgroups are dealt to the 8 XCDs round-robin.  F == 1: blocks b and b + 8 of
  // each group of 16 take chains 2m and 2m + 1 (v-heads 2j, 2j + 1, which read the
  // same K and Q), so the two start together on one XCD and share its L2.  F > 1:
  // in each group of 16 F blocks, the 2 F blocks b = 8 l + x (l = 0 .. 2F - 1) of
  // XCD x take slice l % F of chain 2x + l / F: both chains of a pair, all slices.
  const int chain = V::F == 1 ? (bid & ~15) | ((bid & 7) << 1) | ((bid >> 3) & 1)
                              : (bid / (16 * V::F)) * 16 + 2 * (bid % 8) + (bid / 8) % (2 * V::F) / V::F;
  const int row0 = V::F == 1 ? 0 : ((bid / 8) % V::F) * V::ROWS;
  if (chain >= p.N * p.Hv) return;  // padding of the last group of 16 chains (workgroup-uniform)
  const int h = chain % p.Hv;
  const int seq = pick_sequence<NTHREADS>(sm, p, chain / p.Hv, tid);
  const int hq = h / (p.Hv / p.Hq);
  const int hk = h / (p.Hv / p.Hk);

  int64_t s0 = load_cu(p.cu_seqlens, p.cu_is_64, seq);
  int64_t s1 = load_cu(p.cu_seqlens, p.cu_is_64, seq + 1);
  s0 = s0 < 0 ? 0 : (s0 > p.T ? p.T : s0);
  s1 = s1 < s0 ? s0 : (s1 > p.T ? p.T : s1);
  const int nchunks = int((s1 - s0 + C - 1) / C);

  if (nchunks > 0) {
    // Blocks of T~, N and P that are never written per chunk are read as zeros
    // (strictly-upper blocks, the diagonal blocks of Nh/Nl): clear them once.
    // pick_sequence's last read of its scratch precedes its final barrier.
    const uint4 z = uint4{0u, 0u, 0u, 0u};
    for (int e = tid; e < C * TSTR / 8; e += NTHREADS) {
      reinterpret_cast<uint4*>(sm.P[0])[e] = z;
      reinterpret_cast<uint4*>(sm.P[1])[e] = z;
      reinterpret_cast<uint4*>(sm.Th[0])[e] = z;
      reinterpret_cast<uint4*>(sm.Th[1])[e] = z;
      reinterpret_cast<uint4*>(sm.Tl[0])[e] = z;
      reinterpret_cast<uint4*>(sm.Tl[1])[e] = z;
      if (e < NROWS * TSTR / 8) {
        reinterpret_cast<uint4*>(sm.Nh)[e] = z;
        reinterpret_cast<uint4*>(sm.Nl)[e] = z;
      }
    }
    if (tid < 16) sm.sync[tid] = 0;
    if (V::kHooks && tid == 0) {
      sm.spin_limit = p.spin_limit > 0 ? p.spin_limit : kSpinLimit;
      sm.aborts = p.aborts;
    }
  }
  __syncthreads();  // cleared LDS and counters visible to both roles

  if (wave >= NCW) {
    if (nchunks > 0) {
      if constexpr (V::kLoad) {
        const int64_t tc = (p.T + C - 1) / C;
        const u32x4* tiles = reinterpret_cast<const u32x4*>(p.tiles) + (int64_t(seq) * tc * p.Hv + h) * kTileImage;
        loader_loop<V>(sm, p, tiles, s0, s1, nchunks, h, hq, hk, row0, wave - NCW, lane0);
      } else {
        if constexpr (V::kPipelined) {
          producer_loop_split<V>(sm, p, s0, s1, nchunks, h, hq, hk, row0, wave - NCW, lane0);
        } else {
          producer_loop<V>(sm, p, s0, s1, nchunks, h, hq, hk, row0, wave - NCW, lane0);
        }
      }
    }
    return;
  }

  const int64_t state_head = (int64_t(seq) * p.Hv + h) * D * D;
  const int g = lane0 >> 4, n16 = lane0 & 15;
  if constexpr (V::kTokenSplit) {
    // Token-split consumers: wave w holds column blocks 2w and 2w + 1 (cols k = 16 kt +
    // 4g + i) of the slice's rows v = row0 + n16.
    const int64_t srow = state_head + int64_t(row0 + n16) * D + 32 * wave + 4 * g;
    f32x4 S2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (p.state) {
        const float4 x = *reinterpret_cast<const float4*>(p.state + srow + 16 * j);
        S2[j] = f32x4{x.x, x.y, x.z, x.w};
      } else {
        S2[j] = zero4();
      }
    }
    if (nchunks > 0) {
      consumer_loop_tsplit<V>(sm, p, s0, s1, nchunks, h, row0, wave, lane0, S2);
      if (aborted(sm)) {
        // A hand-off wait gave up: NaN over the slice's outputs (wave w: tokens
        // s0 + 16 (4m + w) + n16) and state.
        const int64_t vstride = int64_t(p.Hv) * D;
        uint16_t* obase = p.out + int64_t(h) * D + row0 + 4 * (lane0 >> 4);
        for (int64_t tok = s0 + 16 * wave + n16; tok < s1; tok += 64)
          *reinterpret_cast<uint2*>(obase + tok * vstride) = uint2{kNaNx2, kNaNx2};
        const float nan = __builtin_nanf("");
        S2[0] = S2[1] = f32x4{nan, nan, nan, nan};
      }
    }
    if (nchunks > 0 || p.state != p.new_state) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        *reinterpret_cast<float4*>(p.new_state + srow + 16 * j) = make_float4(S2[j][0], S2[j][1], S2[j][2], S2[j][3]);
    }
    return;
  }

  // Consumer state slab: rows v = row0 + VW*wave + vrow(vt, n16), cols k = 16*kt + 4g + i.
  f32x4 S[VT][8];
#pragma unroll
  for (int vt = 0; vt < VT; ++vt) {
    const int v = row0 + VW * wave + vrow<VT>(vt, n16);
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
  if (nchunks > 0) {
    consumer_loop<V>(sm, p, s0, s1, nchunks, h, row0, wave, lane0, S);
    if (aborted(sm)) {
      // A hand-off wait gave up: NaN over every output element of this wave (all
      // chunks of the sequence, its state rows of head h) and its state slice.
      const int64_t vstride = int64_t(p.Hv) * D;
      uint16_t* obase = p.out + int64_t(h) * D + row0 + VW * wave + (VT == 2 ? 8 : 4) * (lane0 >> 4);
      for (int64_t tok = s0 + n16; tok < s1; tok += 16) {
        if constexpr (VT == 2) {
          *reinterpret_cast<uint4*>(obase + tok * vstride) = uint4{kNaNx2, kNaNx2, kNaNx2, kNaNx2};
        } else {
          *reinterpret_cast<uint2*>(obase + tok * vstride) = uint2{kNaNx2, kNaNx2};
        }
      }
      const float nan = __builtin_nanf("");
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) S[vt][kt] = f32x4{nan, nan, nan, nan};
    }
  }

  // Final state (for an empty sequence: the initial state, or zeros).
  if (nchunks > 0 || p.state != p.new_state) {
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int v = row0 + VW * wave + vrow<VT>(vt, n16);
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        const f32x4 x = S[vt][kt];
        *reinterpret_cast<float4*>(p.new_state + state_head + int64_t(v) * D + 16 * kt + 4 * g) =
            make_float4(x[0], x[1], x[2], x[3]);
      }
    }
  }
}

// Minimum over the wave (uniform): DPP within each row of 16 lanes, then the four
// row minima.
__device__ __forceinline__ uint32_t wave_min(uint32_t x) {
  x = min(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0xB1, 0xF, 0xF, false)));
  x = min(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x4E, 0xF, 0xF, false)));
  x = min(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x124, 0xF, 0xF, false)));
  x = min(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x128, 0xF, 0xF, false)));
  const uint32_t a = uint32_t(__builtin_amdgcn_readlane(int(x), 0)), b = uint32_t(__builtin_amdgcn_readlane(int(x), 16));
  const uint32_t c = uint32_t(__builtin_amdgcn_readlane(int(x), 32)), d = uint32_t(__builtin_amdgcn_readlane(int(x), 48));
  return min(min(a, b), min(c, d));
}

// Persistent form of the F = 1 kernel, for batches of more chains than CUs: one
// workgroup per CU runs a list of whole chains back to back, so that the next
// chain's first chunk is loaded and prepared while the consumers finish the current
// one (a workgroup per chain pays for that, its start-up and its drain once per
// chain: about three chunk times).  The grid is B = gridDim.x / Hv bins of Hv
// workgroups; workgroup (bin, i) runs v-head h(i) of every sequence of its bin.
// Every workgroup forms the same schedule of the sequences over the bins, so all
// heads of a sequence share one bin and a bin's workgroups share their list: with
// LPT (at most kMaxPersistLpt sequences) longest-processing-time (longest first,
// each onto the least-loaded bin; cost 3 per chunk + 2 per sequence, ties to the
// lower bin), otherwise boustrophedon rounds over the longest-first order.
template <class V, bool LPT>
__global__ __launch_bounds__(V::NTHREADS) void gdn_prefill_persistent_kernel(PrefillArgs p) {
  static_assert(V::kPersist && V::NCW == 4 && V::VT == 2, "persistent kernel: Variant<4, 2, ..., true>");
  constexpr int NCW = V::NCW, VT = V::VT, VW = V::VW, NTHREADS = V::NTHREADS;
  __shared__ PrefillSmem sm;

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bid = blockIdx.x;
  const int nbins = int(gridDim.x) / p.Hv, bin = bid / p.Hv, i = bid % p.Hv;
  // Workgroups are dealt to the 8 XCDs round-robin: with Hv a multiple of 16,
  // workgroups i and i + 8 of a bin (one XCD) take the GQA pair 2j, 2j + 1.
  const int h = p.Hv % 16 == 0 ? (i & ~15) | ((i & 7) << 1) | ((i >> 3) & 1) : i;
  const int hq = h / (p.Hv / p.Hq);
  const int hk = h / (p.Hv / p.Hk);

  // Sequence lengths and starts, then the longest-first order (ties: lower index):
  // for a longest-processing-time list (at most kMaxPersistLpt sequences) in LDS
  // arrays of their own, which consumer wave 0 reads while the first chain runs;
  // for more sequences in the V tile (scratch until the producers stage the first
  // chunk's V).  Chain 0 of bin b is the sequence of rank b either way.
  constexpr bool lpt = LPT;  // p.N <= kMaxPersistLpt
  int* plen = lpt ? sm.plen : reinterpret_cast<int*>(sm.V);
  int* pstart = lpt ? sm.pstart : plen + kMaxSortedSeqs;
  int* porder = lpt ? sm.porder : pstart + kMaxSortedSeqs;
  for (int s = tid; s < p.N; s += NTHREADS) {
    int64_t a = load_cu(p.cu_seqlens, p.cu_is_64, s), b = load_cu(p.cu_seqlens, p.cu_is_64, s + 1);
    a = a < 0 ? 0 : (a > p.T ? p.T : a);
    b = b < a ? a : (b > p.T ? p.T : b);
    plen[s] = int(b - a);
    pstart[s] = int(a);
  }
  // Blocks of T~, N and P that are never written per chunk are read as zeros.
  {
    const uint4 z = uint4{0u, 0u, 0u, 0u};
    for (int e = tid; e < C * TSTR / 8; e += NTHREADS) {
      reinterpret_cast<uint4*>(sm.P[0])[e] = z;
      reinterpret_cast<uint4*>(sm.P[1])[e] = z;
      reinterpret_cast<uint4*>(sm.Th[0])[e] = z;
      reinterpret_cast<uint4*>(sm.Th[1])[e] = z;
      reinterpret_cast<uint4*>(sm.Tl[0])[e] = z;
      reinterpret_cast<uint4*>(sm.Tl[1])[e] = z;
      if (e < NROWS * TSTR / 8) {
        reinterpret_cast<uint4*>(sm.Nh)[e] = z;
        reinterpret_cast<uint4*>(sm.Nl)[e] = z;
      }
    }
    if (tid < 16) sm.sync[tid] = 0;
    if (V::kHooks && tid == 0) {
      sm.spin_limit = p.spin_limit > 0 ? p.spin_limit : kSpinLimit;
      sm.aborts = p.aborts;
    }
    // Every list entry starts as an empty chain, so that no path (a wait for the list
    // that gave up included) reads one that was never written.
    for (int e = tid; e < kMaxPersistList; e += NTHREADS) {
      sm.pseq[e] = 0;
      sm.ps0[e] = 0;
      sm.ps1[e] = 0;
    }
    if (tid == 0) sm.pcount = 1;
  }
  __syncthreads();
  for (int s = tid; s < p.N; s += NTHREADS) {
    const int ls = plen[s];
    int r = 0;
    for (int j = 0; j < p.N; ++j) {
      const int lj = plen[j];
      r += (lj > ls) | ((lj == ls) & (j < s));
    }
    porder[r] = s;
    if (r == bin) {
      sm.pseq[0] = s;
      sm.ps0[0] = pstart[s];
      sm.ps1[0] = pstart[s] + ls;
    }
  }
  if constexpr (!lpt) {
    __syncthreads();  // porder complete
    // Many sequences: boustrophedon over the longest-first order.  Round j of B
    // ranks gives rank jB + b (j even) or jB + B - 1 - b (j odd) to bin b.
    const int cnt = p.N / nbins + (p.N % nbins > (p.N / nbins % 2 == 0 ? bin : nbins - 1 - bin));
    for (int j = 1 + tid; j < cnt; j += NTHREADS) {
      const int r = j * nbins + (j % 2 == 0 ? bin : nbins - 1 - bin);
      const int sj = porder[r];
      sm.pseq[j] = sj;
      sm.ps0[j] = pstart[sj];
      sm.ps1[j] = pstart[sj] + plen[sj];
    }
    if (tid == 0) {
      sm.pcount = cnt;
      sm.sync[kList] = 1;
    }
  }
  __syncthreads();  // chain 0 (with more sequences, the whole list), cleared LDS and counters

  if (wave >= NCW) {
    producer_loop<V>(sm, p, 0, 0, 0, h, hq, hk, 0, wave - NCW, lane0);
    return;
  }

  if (lpt && wave == 0) {
    // The rest of the list, while the producers prepare chain 0's first chunk:
    // longest-processing-time over the bins, longest first, each sequence onto the
    // least-loaded bin (cost 3 per chunk + 2 per sequence; ties to the lower bin;
    // the first B sequences go one per bin, in order).  Lane r holds the cost of the
    // sequence of rank r; lane b < B (at most 64) holds bin b's load.
    const int sr = lane0 < p.N ? porder[lane0] : 0;
    const int lr = lane0 < p.N ? plen[sr] : 0;
    const int cost_r = 3 * (lr / C + (lr % C != 0)) + 2;
    uint32_t load = lane0 < nbins ? 0u : 0xffffffffu;
    int cnt = 0;
    for (int r = 0; r < p.N; ++r) {
      const uint32_t m = wave_min(load);
      const int b = __builtin_ctzll(__ballot(load == m));
      if (lane0 == b) load += uint32_t(__builtin_amdgcn_readlane(cost_r, r));
      if (b == bin) {
        if (lane0 == r && cnt > 0) {
          sm.pseq[cnt] = sr;
          sm.ps0[cnt] = pstart[sr];
          sm.ps1[cnt] = pstart[sr] + lr;
        }
        ++cnt;
      }
    }
    if (lane0 == 0) sm.pcount = cnt;
    signal_count(sm, kList, lane0);
  }

  // Consumers: state rows v = VW*wave + vrow(vt, n16), cols k = 16*kt + 4g + i.
  const int g = lane0 >> 4, n16 = lane0 & 15;
  int nchains = 1;  // chain 0 now; the rest of the list once it is complete
  int u0 = 0;
  for (int k = 0; k < nchains; ++k) {
    const int seq = sm.pseq[k];
    const int64_t s0 = sm.ps0[k], s1 = sm.ps1[k];
    const int nchunks = int((s1 - s0 + C - 1) / C);
    const int64_t state_head = (int64_t(seq) * p.Hv + h) * D * D;
    f32x4 S[VT][8];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int v = VW * wave + vrow<VT>(vt, n16);
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
    if (nchunks > 0) {
      consumer_loop<V>(sm, p, s0, s1, nchunks, h, 0, wave, lane0, S, u0);
      u0 += nchunks;
    }
    // Final state (for an empty sequence: the initial state, or zeros).
    if (nchunks > 0 || p.state != p.new_state) {
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        const int v = VW * wave + vrow<VT>(vt, n16);
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
          const f32x4 x = S[vt][kt];
          *reinterpret_cast<float4*>(p.new_state + state_head + int64_t(v) * D + 16 * kt + 4 * g) =
              make_float4(x[0], x[1], x[2], x[3]);
        }
      }
    }
    if (k == 0) {
      wait_count<V::kHooks>(sm, kList, 1);  // the rest of the list
      nchains = chain_count(sm);
    }
  }
  if (aborted(sm)) {
    // A hand-off wait gave up: NaN over every output element and state element of
    // this wave's rows, in every chain of the workgroup.
    const int64_t vstride = int64_t(p.Hv) * D;
    for (int k = 0; k < nchains; ++k) {
      const int seq = sm.pseq[k];
      const int64_t s0 = sm.ps0[k], s1 = sm.ps1[k];
      uint16_t* obase = p.out + int64_t(h) * D + VW * wave + 8 * (lane0 >> 4);
      for (int64_t tok = s0 + n16; tok < s1; tok += 16)
        *reinterpret_cast<uint4*>(obase + tok * vstride) = uint4{kNaNx2, kNaNx2, kNaNx2, kNaNx2};
      const int64_t state_head = (int64_t(seq) * p.Hv + h) * D * D;
      const float nan = __builtin_nanf("");
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        const int v = VW * wave + vrow<VT>(vt, n16);
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
          *reinterpret_cast<float4*>(p.new_state + state_head + int64_t(v) * D + 16 * kt + 4 * g) =
              make_float4(nan, nan, nan, nan);
      }
    }
  }
}

// Prep kernel of the two-kernel path (few chains).  Item (s R' + r) Hv + h (the
// workgroup index paired as below) prepares chunks r p.prep_chunks .. (r + 1) p.prep_chunks - 1 of sequence s for
// v-head h (R' = ceil(TC / p.prep_chunks)): the producer waves run their loop over
// those chunks and copy each one's T~ hi, T~ lo and P tiles (LDS images) to its
// image in p.tiles; their loads of chunk t + 1 are in flight meanwhile.  Its LDS
// (PrepSmem, one chunk's buffers, no V) lets two workgroups share a CU.  Chunks are
// independent, so all of them are prepared at once; the state pass (Variant<..,
// LOAD = true>) then only copies them.
__global__ __launch_bounds__(PrepVariant::NTHREADS) void gdn_prefill_prep_kernel(PrefillArgs p) {
  constexpr int NTHREADS = PrepVariant::NTHREADS;
  __shared__ PrepSmem sm;
  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tc = (p.T + C - 1) / C;
  const int run = p.prep_chunks;
  const int64_t runs = (tc + run - 1) / run;
  // Workgroups are dealt to the 8 XCDs round-robin: blocks b and b + 8 of each group
  // of 16 take items 2m and 2m + 1 (v-heads 2j and 2j + 1 of one run, which read the
  // same K and Q), so the two share an XCD's L2.
  const int64_t b = blockIdx.x;
  const int64_t bid = (b & ~int64_t(15)) | ((b & 7) << 1) | ((b >> 3) & 1);
  if (bid >= int64_t(p.N) * runs * p.Hv) return;  // padding of the last group of 16 (workgroup-uniform)
  const int h = int(bid % p.Hv);
  const int seq = int(bid / p.Hv / runs), r = int(bid / p.Hv % runs);
  int64_t s0 = load_cu(p.cu_seqlens, p.cu_is_64, seq);
  int64_t s1 = load_cu(p.cu_seqlens, p.cu_is_64, seq + 1);
  s0 = s0 < 0 ? 0 : (s0 > p.T ? p.T : s0);
  s1 = s1 < s0 ? s0 : (s1 > p.T ? p.T : s1);
  const int64_t t0 = int64_t(r) * run;           // first chunk of the run
  const int64_t cs = s0 + t0 * C;
  if (cs >= s1) return;  // the sequence has no chunk t0 (workgroup-uniform)
  const int64_t ce = s1 - cs < int64_t(run) * C ? s1 : cs + int64_t(run) * C;
  const int nchunks = int((ce - cs + C - 1) / C);
  const int hq = h / (p.Hv / p.Hq);
  const int hk = h / (p.Hv / p.Hk);

  // Blocks never written per chunk are zeros (as in the one-kernel path).
  const uint4 z = uint4{0u, 0u, 0u, 0u};
  for (int e = tid; e < C * TSTR / 8; e += NTHREADS) {
    reinterpret_cast<uint4*>(sm.P[0])[e] = z;
    reinterpret_cast<uint4*>(sm.Th[0])[e] = z;
    reinterpret_cast<uint4*>(sm.Tl[0])[e] = z;
    if (e < NROWS * TSTR / 8) {
      reinterpret_cast<uint4*>(sm.Nh)[e] = z;
      reinterpret_cast<uint4*>(sm.Nl)[e] = z;
    }
  }
  if (tid < 16) sm.sync[tid] = 0;
  __syncthreads();
  u32x4* images = reinterpret_cast<u32x4*>(p.tiles) + ((int64_t(seq) * tc + t0) * p.Hv + h) * kTileImage;
  producer_loop<PrepVariant>(sm, p, cs, ce, nchunks, h, hq, hk, 0, wave, lane0, images);
}

// `done`, if not null, is recorded by the launch itself when the kernel completes
// (the kernel's own completion signal; no separate marker in the stream).
template <class V>
hipError_t launch_variant(const PrefillArgs& a, hipStream_t stream, hipEvent_t done = nullptr) {
  const int64_t chains = int64_t(a.N) * a.Hv;
  const int64_t grid = (chains + 15) / 16 * 16 * V::F;
  if (done != nullptr) {
    hipExtLaunchKernelGGL(gdn_prefill_kernel<V>, dim3(unsigned(grid)), dim3(V::NTHREADS), 0, stream, nullptr, done, 0,
                          a);
  } else {
    hipLaunchKernelGGL(gdn_prefill_kernel<V>, dim3(unsigned(grid)), dim3(V::NTHREADS), 0, stream, a);
  }
  return hipGetLastError();
}

int device_cus();

// Batches of more chains than CUs run persistently where they can: a workgroup per
// CU, Hv dividing the CUs into B <= 64 bins, at most kMaxSortedSeqs sequences and
// kMaxPersistList per bin.
bool persistent_batch(const PrefillArgs& a) {
  const int cus = device_cus();
  if (cus % a.Hv != 0 || cus / a.Hv > 64 || a.N > kMaxSortedSeqs || int64_t(a.N) * a.Hv <= cus) return false;
  const int bins = cus / a.Hv;
  return (a.N + bins - 1) / bins <= kMaxPersistList;
}

template <class V>
hipError_t launch_persistent(const PrefillArgs& a, hipStream_t stream) {
  if (a.N <= kMaxPersistLpt) {
    hipLaunchKernelGGL((gdn_prefill_persistent_kernel<V, true>), dim3(unsigned(device_cus())), dim3(V::NTHREADS), 0,
                       stream, a);
  } else {
    hipLaunchKernelGGL((gdn_prefill_persistent_kernel<V, false>), dim3(unsigned(device_cus())), dim3(V::NTHREADS), 0,
                       stream, a);
  }
  return hipGetLastError();
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static std::atomic<int> cus[64];  // 0 until queried; racing first queries store the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace

// Scratch of gdn_prefill_no_alloc: the chunk images of the two-kernel path, for
// callers that cannot allocate.  Each device that loads the library holds its own
// copy until the process ends; every call on a device shares it.
static __device__ __align__(256) uint8_t scratch[kPrefillScratchBytes];

// Scratch of the drop-in gdn_prefill's two-kernel path (long sequences, below):
// its own array, so that no call of gdn_prefill_no_alloc, captured or not, shares it.
static __device__ __align__(256) uint8_t dropin_scratch[kPrefillDropinScratchBytes];

namespace {
constexpr int kMaxDevices = 64;

// Per device and scratch array: the array's device address (looked up once, with
// the device current: in host code the array's name is a host-side stand-in), the
// event that follows the last launch using it, and the lock that orders the
// check-launch-record sequence between host threads.  Created on first use and
// kept until the process ends, like the array itself.
struct OrderedScratch {
  std::mutex lock;
  void* addr = nullptr;
  hipEvent_t done = nullptr;
  bool used = false;
};
OrderedScratch g_dropin[kMaxDevices];
OrderedScratch g_no_alloc[kMaxDevices];

// Launches the two-kernel path of `a` with its chunk images in the scratch array
// `symbol`, ordered after the previous launch that used the array on this device:
// the stream waits for that launch's event, and the state pass records the event
// again as it completes.  If the launch fails after the prep kernel was enqueued,
// the event is recorded behind it all the same, so the next launch still waits for
// the orphaned kernel.
hipError_t launch_ordered(const PrefillArgs& a, hipStream_t stream, OrderedScratch* table, const void* symbol) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  OrderedScratch& d = table[dev];
  std::lock_guard<std::mutex> guard(d.lock);
  if (d.addr == nullptr) {
    e = hipGetSymbolAddress(&d.addr, symbol);
    if (e != hipSuccess) return e;
  }
  if (d.done == nullptr) {
    e = hipEventCreate(&d.done);
    if (e != hipSuccess) return e;
  }
  if (d.used) {
    e = hipStreamWaitEvent(stream, d.done, 0);
    if (e != hipSuccess) return e;
  }
  PrefillArgs b = a;
  b.tiles = static_cast<uint16_t*>(d.addr);
  e = launch_prefill(b, stream, d.done);  // the state pass records `done` as it completes
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipEventRecord(d.done, stream);
  }
  d.used = true;
  return e;
}

bool stream_capturing(hipStream_t stream, hipError_t* err) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  *err = hipStreamIsCapturing(stream, &capture);
  return *err == hipSuccess && capture != hipStreamCaptureStatusNone;
}
}  // namespace

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.  In host code `scratch` names a
// host-side stand-in, so kernels and copies must use this address instead.
hipError_t prefill_scratch(void** ptr) {
  static std::atomic<void*> addr[kMaxDevices];  // null until looked up; racing lookups store the same value
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev].store(p, std::memory_order_release);
  }
  *ptr = p;
  return hipSuccess;
}

int64_t prefill_static_device_bytes() {
  return int64_t(sizeof(scratch)) + int64_t(sizeof(dropin_scratch)) + int64_t(sizeof(gdn_prefill_giveup_count));
}

// The drop-in gdn_prefill.  A batch of N sequences averaging at least
// kDropinTwoKernelTokens tokens (T >= kDropinTwoKernelTokens N), whose chains the
// launcher splits 4 or 8 ways, runs on the two-kernel path (each chunk prepared once)
// in dropin_scratch when its images fit; everything else, and any launch on a stream
// that is being captured into a graph, runs launch_prefill as is.  (The host sees N
// and T, not the lengths; measured, one kernel against two, µs: [2048, 2048] 111.2 /
// 99.2, [300, 4000] 189.4 / 150.2, [1000, 1100] 62.2 / 59.8, [900, 1200, 100, 3000]
// at 16 v-heads 142.2 / 114.0, and below the threshold [600, 700] 42.5 / 42.4,
// [512] x 4 at 16 v-heads 32.7 / 36.9.)  Launches on the scratch are ordered on the
// device (launch_ordered), so calls on any streams stay correct, and calls on one
// stream wait for nothing they would not wait for anyway.
hipError_t launch_prefill_dropin(const PrefillArgs& a, hipStream_t stream) {
  const int64_t need =
      a.N >= 1 && a.T >= kDropinTwoKernelTokens * a.N ? prefill_workspace_bytes(a.N, a.T, a.Hv) : 0;
  if (need <= 0 || need > kPrefillDropinScratchBytes || a.spin_limit != 0 || a.ready_chunks != 0 ||
      a.aborts != nullptr || a.tiles != nullptr)
    return launch_prefill(a, stream);
  hipError_t e = hipSuccess;
  if (stream_capturing(stream, &e)) return launch_prefill(a, stream);
  if (e != hipSuccess) return e;
  return launch_ordered(a, stream, g_dropin, HIP_SYMBOL(dropin_scratch));
}

// gdn_prefill_no_alloc: the two-kernel path in `scratch` for batches that take it.
// On a stream that is not being captured, launches are ordered on the device like
// the drop-in's (their own event), so eager calls on any streams stay correct.  A
// launch captured into a graph cannot wait for that event: its replays and any other
// use of the array on the device must not overlap.
hipError_t launch_prefill_no_alloc(const PrefillArgs& a, hipStream_t stream) {
  const int64_t need = prefill_workspace_bytes(a.N, a.T, a.Hv);
  if (need <= 0) return launch_prefill(a, stream);
  if (need > kPrefillScratchBytes) return hipErrorInvalidValue;
  hipError_t e = hipSuccess;
  if (stream_capturing(stream, &e)) {
    PrefillArgs b = a;
    e = prefill_scratch(reinterpret_cast<void**>(&b.tiles));
    if (e != hipSuccess) return e;
    return launch_prefill(b, stream);
  }
  if (e != hipSuccess) return e;
  return launch_ordered(a, stream, g_no_alloc, HIP_SYMBOL(scratch));
}

// Reads (and with `reset` clears) this device's give-up count, after
// synchronising the device so that every launch so far has finished.
hipError_t prefill_giveups(uint64_t* count, bool reset) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  unsigned int v = 0;
  e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(gdn_prefill_giveup_count), sizeof(v));
  if (e != hipSuccess) return e;
  *count = v;
  if (reset) {
    const unsigned int z = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(gdn_prefill_giveup_count), &z, sizeof(z));
  }
  return e;
}

#ifndef GDN_PREFILL_MAX_SPLIT
#define GDN_PREFILL_MAX_SPLIT 8
#endif

namespace {
// Chains are split F ways (F a power of two, at most GDN_PREFILL_MAX_SPLIT)
// while the split grid still fits one workgroup per CU.
int split_factor(int64_t chains) {
  const int64_t cus = device_cus();
  int F = 1;
  while (F < GDN_PREFILL_MAX_SPLIT && chains * 2 * F <= cus) F *= 2;
  return F;
}

}  // namespace

int64_t prefill_work_items(int64_t chains) {
  if (chains <= 0) return 0;
  const int F = split_factor(chains);
  const int64_t grid = (chains + 15) / 16 * 16 * F;
  switch (F) {
    case 1: return grid * SplitVariant1<false>::NTHREADS;
    case 2: return grid * SplitVariant2<false>::NTHREADS;
    case 4: return grid * SplitVariant4<false>::NTHREADS;
    default: return grid * SplitVariant8<false>::NTHREADS;
  }
}

namespace {
// Largest workspace the two-kernel path uses; bigger batches take one kernel.
constexpr int64_t kMaxWorkspaceBytes = int64_t(2) << 30;
// Images above this size are read back mostly from HBM by the state pass.
constexpr int64_t kDeepImageBytes = int64_t(64) << 20;
}  // namespace

// Batches split 4 or 8 ways repeat the producer work in every slice of a chain and
// are bound by it; the two-kernel path prepares each chunk once, all chunks in
// parallel, and its state pass (no producer code: 16-row consumers fit in the
// registers) runs at the consumers' pace.  Batches split 2 ways lose more to the
// extra pass than they gain, and unsplit ones keep producers and consumers busy
// on the same CUs.
int64_t prefill_workspace_bytes(int N, int64_t T, int Hv) {
  if (N <= 0 || Hv <= 0 || T <= 0 || split_factor(int64_t(N) * Hv) < 4) return 0;
  const int64_t images = int64_t(N) * ((T + C - 1) / C) * Hv;
  if (images > INT32_MAX) return 0;
  const int64_t bytes = images * kTileImage * 16;
  return bytes <= kMaxWorkspaceBytes ? bytes : 0;
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream, hipEvent_t done) {
  const int F = split_factor(int64_t(a.N) * a.Hv);
  // Launches that use the testing hooks get kernels with the hooks compiled in;
  // production launches keep them out of the device code.
  if (a.spin_limit != 0 || a.ready_chunks != 0 || a.aborts != nullptr) {
    if (persistent_batch(a)) return launch_persistent<PersistVariant<true>>(a, stream);
    switch (F) {
      case 1: return launch_variant<SplitVariant1<true>>(a, stream);
      case 2: return launch_variant<SplitVariant2<true>>(a, stream);
      case 4: return launch_variant<SplitVariant4<true>>(a, stream);
      default: return launch_variant<SplitVariant8<true>>(a, stream);
    }
  }
  if (a.tiles != nullptr && prefill_workspace_bytes(a.N, a.T, a.Hv) > 0) {
    // Runs of consecutive chunks per prep workgroup, about two workgroups per CU
    // for the batch's chunks (at most T / C + N of them).
    const int64_t tc = (a.T + C - 1) / C;
    const int64_t chunks = a.T / C + a.N < a.N * tc ? a.T / C + a.N : a.N * tc;
    const int64_t slots = 2 * int64_t(device_cus());
    const int64_t run = (chunks * a.Hv + slots - 1) / slots;
    PrefillArgs b = a;
    b.prep_chunks = int(run < 1 ? 1 : run > tc ? tc : run);
    const int64_t grid = (int64_t(a.N) * ((tc + b.prep_chunks - 1) / b.prep_chunks) * a.Hv + 15) / 16 * 16;
    hipLaunchKernelGGL(gdn_prefill_prep_kernel, dim3(unsigned(grid)), dim3(PrepVariant::NTHREADS), 0, stream, b);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (F == 4) return launch_variant<Variant<2, 1, false, true>>(a, stream, done);
    // Split 8 ways, images beyond what the caches keep between the two kernels are
    // loaded two chunks ahead (one sequence, 32 v-heads, 19,200-byte images: 12,288
    // tokens, 118 MB of images, 420.1 -> 396.9 us; 10,500 tokens 349.8 -> 333.8;
    // 8,192 tokens, 79 MB, 255.7 -> 252.5; 6,000 tokens, 58 MB, 187.8 -> 188.0).
    // Split 4 ways it measured no change (two 4,096-token sequences, images of whole
    // tiles: 186.2 -> 185.8 us).
    if (prefill_workspace_bytes(a.N, a.T, a.Hv) > kDeepImageBytes)
      return launch_variant<Variant<4, 1, false, true, 4, false, true, true>>(a, stream, done);
    return launch_variant<Variant<4, 1, false, true, 4, false, true>>(a, stream, done);
  }
  // Split chains use 16-row consumer waves (VT = 1), whose per-chunk chain is
  // shorter than a 32-row wave's.  Unsplit chains (F = 1) keep four 32-row waves:
  // eight 16-row waves and the four producers would exceed the register file.
  if (persistent_batch(a)) return launch_persistent<PersistVariant<false>>(a, stream);
  switch (F) {
    case 1: return launch_variant<SplitVariant1<false>>(a, stream);
    case 2: return launch_variant<SplitVariant2<false>>(a, stream);
    case 4: return launch_variant<SplitVariant4<false>>(a, stream);
    default: return launch_variant<SplitVariant8<false>>(a, stream);
  }
}

}  // namespace gdn


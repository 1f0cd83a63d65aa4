// 2-simplicial attention forward for 16-bit operands on gfx950 (CDNA4),
// written as flash attention over key PAIRS: the kernel behind
// mf_simplicial_fwd for bf16/fp16, head_dim <= 64 (a multiple of 8) and
// tokens <= kMaxN.
//
// Math (simplicial_attention.py:161-180,304-344; triton_simplicial_attention.py:115-329):
//   S_i[j,k] = sum_d q_i[d] k1_j[d] k2_k[d]
//   P_i      = softmax over valid (j,k) of S_i
//   out_i[d] = sum_{j,k} P_i[j,k] v1_j[d] v2_k[d],   lse_i = log sum_{j,k} exp(S_i[j,k])
// Read the valid pairs p = (j,k) as keys with key vector W_p = k1_j (.) k2_k
// and value vector Z_p = v1_j (.) v2_k: then S = Q W^T and out = softmax(S) Z,
// plain attention over nk^2 keys whose tiles are formed on the fly.
//
// One launch.  A persistent grid of 2 workgroups per CU; each workgroup
// first scans every molecule's two byte masks (valid keys, valid queries)
// straight from global memory, ranks the molecules by cost and enumerates the
// units (molecule b, head h, query group g) in that order, longest first --
// every workgroup derives the same list.  Workgroup w takes position w;
// after that a workgroup that finishes a unit claims the next position with
// one device-scope atomic on a counter in the caller's workspace (each unit
// makes one claim, so the claim that returns the unit count minus one is the
// launch's last, and its workgroup puts the counter back to 0: every launch,
// graph replays included, starts from 0).  A query group is
// at most 48 valid queries (3 tiles of 16); molecules with more than 48
// queries use groups of 32.  Each workgroup zeroes the rows of padded
// queries of a static share of (b, h) after its first unit.
//
// Per unit the workgroup stages the unit's valid key rows (compacted) into
// LDS as fp16 scaled by powers of two: K1s, K2s row-major, V1s, V2s as
// [row][r16][dt] (the ND = DP/16 halves of columns r16, 16+r16, ... side by
// side), and the group's query rows Qs = q log2(e) 2^sq.  The scales
// normalise max|K1|, max|K2|, max|V1|, max|V2| into [1, 2), so every pair
// product is a normal fp16 number and one v_pk_mul_f16 forms two of them;
// sq = -(s1 + s2) keeps S in log2 units.  Keys beyond kCap are taken in
// (j block, k block) pairs of kCap keys.
//
// The four waves split the iterations (16-key tile kt of k, pair of rows
// j0, j0+1) of the unit.  Per iteration and wave (QT query tiles):
//   W      = K1s[j] (.) K2s[k0 + r16]            (A operand: pair = row, d = K)
//   GEMM1  S^T[pair][i] = W Q^T                   (MFMA 16x16x32 f16, 2 QT per j)
//   P      = fp16(2^S)                            (B operand of GEMM2 straight from
//                                                  the accumulators: keys 4g+r of j0
//                                                  and of j0+1 are K 8g..8g+7)
//   Z      = V1s[j] (.) V2s[k0 + 4g + r]          (A operand: d = row, pair = K)
//   GEMM2  O^T[d][i] += Z^T P                     (MFMA, ND QT per iteration)
//   L[i]  += 1^T P                                (one MFMA per query tile, A = 1
//                                                  at the valid keys)
// Padded keys (k >= nk) and the padding row j0+1 = nk have zero K and V rows:
// their P is finite, Z = 0 removes them from O and the ones operand from L.
// pair_valid clears P bit by bit.
//
// No running maximum in the common case.  With m_d = max_j |k1_j[d]| and
// n_d = max_k |k2_k[d]|, |S_i[j,k]| <= U_i = sum_d |q'_i[d]| m_d n_d.  When
// U_i <= kBoundLimit for every query of the unit (and the query scale is
// representable), P = 2^S lies in [2^-U, 2^U], inside the normal fp16 range,
// and softmax is invariant to the missing offset.  Otherwise a single-block
// unit whose bounds are at most kShiftMax first takes one shifted pass,
// P = 2^(S - m_i) with m_i = max(U_i - kShiftTop, 0), kept when every shifted
// query's denominator reaches kMinMass.  Failing that, the unit takes the
// exact offsets: two passes, the maximum m_i of the valid logits (GEMM1
// only), then P = 2^(S - m_i) with S rescaled to log2 units (the query scale
// is then normalised on its own: sq = 1 - exponent(max|q'|)); with the bias,
// one pass whose offsets follow the running maxima (O and L rescaled when a
// tile's maximum passes the offset by more than kOnlineSlack), the waves'
// partials moved to the largest of their offsets at the end.
#include <cmath>
#include <type_traits>

#include "mf_common.h"

namespace mf {
namespace spair {

// Waves per workgroup (4, two workgroups per CU: two waves on every SIMD, which the pair loop needs to
// overlap MFMA and VALU), queries per unit and keys per staged block.  The bias instantiations stage 80-key
// blocks (molecules of up to 80 atoms in one block) with 32 staged query rows, so that their bias operands
// fit beside a second workgroup's LDS.
template <bool BIAS>
struct Waves {
  static constexpr int kCount = 4;
  // queries per unit: 3 tiles; 2 with the bias, whose operands leave no room for a third at 256
  // registers per wave
  static constexpr int kGroup = BIAS ? 32 : 48;
  static constexpr int kMaxQ = kGroup;          // staged query rows
  static constexpr int kCap = BIAS ? 80 : 128;  // keys per staged block (a multiple of 16)
  static constexpr int kPVW = (kCap + 31) / 32;  // pair-valid words per staged row
};
constexpr int kRedWaves = 4;          // partial-output slots of the final reduction
constexpr int kMaxBatch = 256;        // molecules per launch
constexpr int kMaxN = 512;            // tokens
constexpr float kBoundLimit = 13.5f;  // fast path bound on |S| (log2 units)
constexpr float kQLimit = 8192.0f;    // fast path bound on max |Qs|
// Shifted one-pass mode (a unit past the fast-path bound, single key block): query i takes the offset
// m_i = max(B_i - kShiftTop, 0) from its own bound |S| <= B_i (log2 units), so every 2^(S - m_i) <= 2^14 fits
// fp16; the pass is kept when every shifted query's denominator reaches kMinMass (then terms lost to fp16
// underflow, at most one 2^-25 per pair, stay below 2^-10 of it), else the unit reruns the exact way.
// Bounds above kShiftMax (large or masking-scale terms, whose shifted pass mostly fails and costs a pass) go
// to the exact way at once.  The exact way: the maximum of the valid logits, then the main pass (a max pass
// and a pass with those offsets); the bias instantiations take one pass with running offsets (kOnline).
constexpr float kShiftTop = 14.0f;
constexpr float kShiftMax = 24.0f;
constexpr float kMinMass = 0.25f;

// kOnline: one pass with a running offset per query (raised, with the query's O and L rescaled, when a tile's
// maximum passes it by more than kOnlineSlack), for units that need the exact offsets
enum Mode { kFast = 0, kSlow = 1, kMax = 2, kOnline = 3 };
constexpr float kOnlineSlack = 8.0f;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

struct Params {
  const void* q;
  const void* k1;
  const void* v1;
  const void* k2;
  const void* v2;
  const uint8_t* qv;
  const uint8_t* pkv;
  const uint8_t* pv;
  void* out;
  float* out_f32;
  float* lse;
  unsigned int* counter;  // claims of this launch (0 at launch start and end)
  int B, H, N, D;
  // factorized bias S[j,k] += gate_i (u_ij + v_ik + w_jk): u, v, w [B*H, N, N] and gate [B*H, N] in
  // bias_dtype (the BIAS instantiations only)
  const void* bu;
  const void* bv;
  const void* bw;
  const void* bg;
  int bias_dtype;
  // element strides {batch, head, token} of q, of k1 / v1 / k2 / v2, and of out (d is unit-stride);
  // the contiguous [B*H, N, D] layout unless the caller passed others.  32-bit (the host refuses larger
  // ones): the kernel is short of scalar registers, and 64-bit strides cost it more spills.
  int qs_b, qs_h, qs_n;
  int ks_b, ks_h, ks_n;
  int os_b, os_h, os_n;
};

// The claim counter in the caller's workspace (its own 128-byte line).  It
// must be 0 before the first launch; every launch leaves it 0.
constexpr size_t kSyncBytes = 256;

// Claim state of a workgroup (LDS): claimed != 0 when the unit just run
// claimed the next position, next = that position.
struct ClaimState {
  int claimed;
  int next;
};

// Thread 0's claim: position G + ticket.  A launch of `total` units makes
// exactly `total` claims (one per unit run, the last of each workgroup's
// failing), which return 0 .. total - 1; the one that returns total - 1 is
// the last, so no claim of this launch can follow its reset of the counter.
__device__ __forceinline__ int claimed_position(unsigned int* counter, unsigned int ticket, int total) {
  if (int(ticket) == total - 1) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return int(gridDim.x) + int(ticket);
}

// LDS layout (bytes) for padded head dim DP.
template <int DP, bool BIAS>
struct Lay {
  static constexpr int kWaves = Waves<BIAS>::kCount;
  static constexpr int kCap = Waves<BIAS>::kCap;
  static constexpr int kMaxQ = Waves<BIAS>::kMaxQ;
  static constexpr int kPVW = Waves<BIAS>::kPVW;
  static constexpr int RQ = Waves<BIAS>::kGroup;  // query rows of a reduction slot
  static constexpr int RB = DP * 2;  // bytes per staged fp16 row
  static constexpr int kK1 = 0;
  static constexpr int kK2 = kK1 + kCap * RB;
  static constexpr int kV1 = kK2 + kCap * RB;
  static constexpr int kV2 = kV1 + kCap * RB;
  static constexpr int kQ = kV2 + kCap * RB;
  static constexpr int kPV = kQ + kMaxQ * RB;             // u32 [kCap][kPVW] pair-valid bits
  static constexpr int kInfo = kPV + kCap * kPVW * 4;     // u32 [kMaxBatch] molecule info
  static constexpr int kPre = kInfo + kMaxBatch * 4;     // int [kMaxBatch + 4] unit prefix by rank
  static constexpr int kOrder = kPre + (kMaxBatch + 4) * 4;  // u16 [kMaxBatch] molecule of each rank
  static constexpr int kKidx = kOrder + kMaxBatch * 2;   // u16 [kMaxN] valid key atoms
  static constexpr int kQidx = kKidx + kMaxN * 2;        // u16 [kMaxN] valid query atoms
  // column maxima float [kWaves][2][DP]; aliased by the molecule costs
  // (schedule) and by the per-wave query maxima (two-pass mode)
  static constexpr int kColBytes = kWaves * 2 * DP * 4 > kMaxBatch * 4 ? kWaves * 2 * DP * 4 : kMaxBatch * 4;
  static constexpr int kCol = kQidx + kMaxN * 2;
  static constexpr int kMn = kCol + (kColBytes > kWaves * kMaxQ * 4 ? kColBytes : kWaves * kMaxQ * 4);
  static constexpr int kG = kMn + DP * 4;       // float [kWaves][4] |V1|, |V2|, |q| maxima
  static constexpr int kScal = kG + kWaves * 4 * 4;  // int [8] scale exponents, slow flag, no-shift flag
  static constexpr int kM = kScal + 8 * 4;      // float [kMaxQ] two-pass maxima (log2 units)
  static constexpr int kClaim = kM + kMaxQ * 4;  // ClaimState
  static constexpr int kTotal = kClaim + int(sizeof(ClaimState));
  // after the pair loop: partial outputs float [kRedWaves][RQ][RS] and
  // denominators float [kRedWaves][RQ], over K1s .. V2s, Qs and the pair bits
  // (none of them is read after the pair loop)
  static constexpr int RS = DP + 4;
  static constexpr int kRed = 0;
  static constexpr int kRedL = kRed + kRedWaves * RQ * RS * 4;
  static_assert(kRedL + kRedWaves * RQ * 4 <= kInfo, "reduction area must fit in the staging area");
  // BIAS instantiations, after the above: fp16 bias operands of the unit's (j block, k block)
  //   BU [kCap][kMaxQ]     c_i u_ij (row j, query i)
  //   BW [kCap][kCap]      w_jk
  //   BV [kMaxQ][kVS]      c_i v_ik at half k + 2 (halves 0, 1 and past the keys read as masked)
  //   BG float [kMaxQ]     c_i = log2(e) 2^E gate_i; then per-query |u|, |v| maxima and the block |w| maximum
  static constexpr int kVS = kCap + 16;
  static constexpr int kBU = (kTotal + 15) & ~15;
  static constexpr int kBW = kBU + kCap * kMaxQ * 2;
  static constexpr int kBV = kBW + kCap * kCap * 2;
  static constexpr int kBG = kBV + kMaxQ * kVS * 2;
  static constexpr int kBMax = kBG + kMaxQ * 4;  // float [2][kMaxQ] |u|, |v| maxima, then |w|
  static constexpr int kTotalBias = kBMax + (2 * kMaxQ + 1) * 4;
};

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pkmul(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, a) * __builtin_bit_cast(h2_t, b));
}
__device__ __forceinline__ uint4 pkmul4(uint4 a, uint4 b) {
  return uint4{pkmul(a.x, b.x), pkmul(a.y, b.y), pkmul(a.z, b.z), pkmul(a.w, b.w)};
}
// (a.lo * w.h, a.hi * w.h) with w.h the half HI of w
template <int HI>
__device__ __forceinline__ uint32_t pkmul_splat(uint32_t a, uint32_t w) {
  const h2_t x = __builtin_bit_cast(h2_t, w);
  const h2_t s = HI ? h2_t{x.y, x.y} : h2_t{x.x, x.x};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, a) * s);
}
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{lo, hi}, h2_t));
}
__device__ __forceinline__ mf_f32x4 mfma(uint4 a, uint4 b, mf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf_f16x8, a), __builtin_bit_cast(mf_f16x8, b), c,
                                                0, 0, 0);
}

template <typename T>
__device__ __forceinline__ float elem_lo(uint32_t w) {
  if constexpr (std::is_same<T, __bf16>::value) return __uint_as_float(w << 16);
  else return float(__builtin_bit_cast(h2_t, w).x);
}
template <typename T>
__device__ __forceinline__ float elem_hi(uint32_t w) {
  if constexpr (std::is_same<T, __bf16>::value) return __uint_as_float(w & 0xffff0000u);
  else return float(__builtin_bit_cast(h2_t, w).y);
}
// the 8 elements of a 16-byte chunk as floats
template <typename T>
__device__ __forceinline__ void unpack8(uint4 u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f[2 * p] = elem_lo<T>(w[p]);
    f[2 * p + 1] = elem_hi<T>(w[p]);
  }
}

// Maximum over the lanes l ^ OFF, l ^ OFF/2, ..., l ^ LAST (log2 NV steps)
// of NV values per lane, scattered: each step keeps half of the values, so
// the lane ends with the maximum of value idx.
template <int NV, int OFF, int LAST>
__device__ __forceinline__ float reduce_scatter_max(const float (&v)[NV], int lane, int& idx) {
  if constexpr (NV == 1) {
    // remaining steps reduce the single value
    float r = v[0];
#pragma unroll
    for (int off = OFF; off >= LAST; off >>= 1) r = fmaxf(r, __shfl_xor(r, off, 64));
    idx = 0;
    return r;
  } else if constexpr (OFF < LAST) {
    // no lanes left: reduce locally
    float r = v[0];
#pragma unroll
    for (int i = 1; i < NV; ++i) r = fmaxf(r, v[i]);
    idx = -1;
    return r;
  } else {
    const bool up = (lane & OFF) != 0;
    float k[NV / 2];
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      const float send = up ? v[i] : v[i + NV / 2];
      const float keep = up ? v[i + NV / 2] : v[i];
      k[i] = fmaxf(keep, __shfl_xor(send, OFF, 64));
    }
    int sub;
    const float r = reduce_scatter_max<NV / 2, OFF / 2, LAST>(k, lane, sub);
    idx = (up ? NV / 2 : 0) + sub;
    return r;
  }
}

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a),
                                                                __builtin_bit_cast(u16x2_t, b)));
}
// Cross-lane reductions on VALU (DPP and v_permlane*_swap) instead of
// ds_bpermute.  group_reduce<G>: every lane gets op over its aligned group of
// G consecutive lanes (quad permutes; then the half-row and row mirrors,
// which pair a lane with the other half of its group once each half holds
// its own total; then the 16- and 32-lane swaps, whose two results are the
// lane's value and its partner's, in some order).  stride_reduce<S>: op over
// the lanes l' = l mod S (row rotations by 4 and 8 within rows of 16, then
// the swaps).  Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_peer(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), CTRL, 0xf, 0xf, false));
}
template <typename Op>
__device__ __forceinline__ uint32_t swap16_op(uint32_t v, Op op) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return op(uint32_t(r[0]), uint32_t(r[1]));
}
template <typename Op>
__device__ __forceinline__ uint32_t swap32_op(uint32_t v, Op op) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return op(uint32_t(r[0]), uint32_t(r[1]));
}
template <int G, typename Op>
__device__ __forceinline__ uint32_t group_reduce(uint32_t v, Op op) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
  if constexpr (G >= 2) v = op(v, dpp_peer<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  if constexpr (G >= 4) v = op(v, dpp_peer<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  if constexpr (G >= 8) v = op(v, dpp_peer<0x141>(v));  // row_half_mirror
  if constexpr (G >= 16) v = op(v, dpp_peer<0x140>(v)); // row_mirror
  if constexpr (G >= 32) v = swap16_op(v, op);
  if constexpr (G >= 64) v = swap32_op(v, op);
  return v;
}
template <int S, typename Op>
__device__ __forceinline__ uint32_t stride_reduce(uint32_t v, Op op) {
  static_assert(S == 4 || S == 8, "stride");
  if constexpr (S == 4) v = op(v, dpp_peer<0x124>(v));  // row_ror:4
  v = op(v, dpp_peer<0x128>(v));                        // row_ror:8
  v = swap16_op(v, op);
  return swap32_op(v, op);
}
struct PkMaxU16 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return pk_max_u16(a, b); }
};
struct MaxF32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }
};
struct AddF32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }
};
struct AddI32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; }
};
struct MaxI32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return uint32_t(max(int(a), int(b))); }
};
struct MinI32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return uint32_t(min(int(a), int(b))); }
};

// |x| from the 16-bit pattern of x with the sign cleared
template <typename T>
__device__ __forceinline__ float mag_to_float(uint32_t m) {
  if constexpr (std::is_same<T, __bf16>::value) return __uint_as_float(m << 16);
  else return float(__builtin_bit_cast(_Float16, uint16_t(m)));
}

// Exponent s with x 2^s in [1, 2) (0 for x == 0 or not finite).
__device__ __forceinline__ int norm_exp(float x) {
  if (!(x > 0.0f) || !(x < INFINITY)) return 0;
  int e;
  (void)frexpf(x, &e);
  return 1 - e;
}

// Molecule info word: nk | nq << 11 | kpre << 30 | qpre << 31 (kpre / qpre:
// the valid keys / queries are exactly the prefix 0..n-1).
constexpr uint32_t kKPre = 1u << 30;
constexpr uint32_t kQPre = 1u << 31;
__device__ __forceinline__ int info_nk(uint32_t w) { return int(w & 0x7ffu); }
__device__ __forceinline__ int info_nq(uint32_t w) { return int((w >> 11) & 0x7ffu); }

// Query groups of a molecule with nk valid keys and nq valid queries: one
// group of up to GQ (48, or 32 with the bias), else groups of 32; molecules
// with more than kCap keys (taken in key blocks) use groups of 16, one query
// tile.
template <int GQ, int kCap>
__device__ __forceinline__ int group_size(int nk, int nq) {
  if (nk > kCap) return 16;
  return nq <= GQ ? GQ : 32;
}
template <int GQ, int kCap>
__device__ __forceinline__ int num_groups(int nk, int nq) {
  if (nq <= 0) return 0;
  if (nk > kCap) return (nq + 15) >> 4;
  return nq <= GQ ? 1 : (nq + 31) >> 5;
}

// i / d for 0 <= i, d and i + d < 2^21: (i + 1/2) / d is at least 1/(2d)
// away from an integer, more than the error of the float reciprocal.
__device__ __forceinline__ int div_small(int i, int d) {
  return int((float(i) + 0.5f) * __builtin_amdgcn_rcpf(float(d)));
}

// dst[r] = the atom of valid rank r in a mask row (one wave).
__device__ __forceinline__ void write_ranks(const uint8_t* row, int N, uint16_t* dst, int lane) {
  const unsigned long long below = (1ull << lane) - 1ull;
  int run = 0;
  for (int t0 = 0; t0 < N; t0 += 64) {
    const int t = t0 + lane;
    const bool ok = t < N && row[t] != 0;
    const unsigned long long bal = __ballot(ok);
    if (ok) dst[run + __popcll(bal & below)] = uint16_t(t);
    run += __popcll(bal);
  }
}

// ---------------------------------------------------------------------------
// pair loop of one wave over its share of a staged block
// ---------------------------------------------------------------------------
template <int DP>
struct Shape {
  static constexpr int NCH = DP / 32;  // 32-wide d chunks (GEMM1 K steps)
  static constexpr int ND = DP / 16;   // 16-wide d tiles (GEMM2 M tiles)
};

// Pair-valid mask (0xffff per valid half) of keys k0 + 4g + {2 s, 2 s + 1}
// of row j.
__device__ __forceinline__ uint32_t pv_mask(uint32_t bits4, int s) {
  return ((bits4 >> (2 * s)) & 1u ? 0x0000ffffu : 0u) | ((bits4 >> (2 * s + 1)) & 1u ? 0xffff0000u : 0u);
}

// The first QT of the MQ query tiles held in registers are in use.
//
// BIAS: GEMM1 gets one more 32-wide K step per (row, query tile) whose
// operands carry the factorized bias in log2 units (c_i = log2(e) 2^E gate_i):
//   A[pair p][K]: K = 0 -> 1, K = 1 -> w[j][k0 + p], K = 2 + t -> (p == t), t < 16
//   B[K][i]     : K = 0 -> c_i u[i][j], K = 1 -> c_i, K = 2 + t -> c_i v[i][k0 + t]
// so the accumulator gains c_i (u_ij + w_jk + v_ik) for pair (j, k0 + p).
template <int DP, int QT, int MODE, bool HAS_PV, bool BIAS, int MQ>
__device__ __forceinline__ void pair_loop(const unsigned char* smem, int nkj, int nkk,
                                          const uint4 (&qop)[MQ][DP / 32], float (&negm)[MQ], float sc,
                                          mf_f32x4 (&O)[DP / 16][MQ], mf_f32x4 (&L)[MQ], float (&mloc)[MQ], int wave,
                                          int g, int r16) {
  constexpr int W = Waves<BIAS>::kCount;
  using Ly = Lay<DP, BIAS>;
  constexpr int kCap = Ly::kCap;
  constexpr int RB = Ly::RB;
  constexpr int NCH = Shape<DP>::NCH;
  constexpr int ND = Shape<DP>::ND;
  const unsigned char* K1s = smem + Ly::kK1;
  const unsigned char* K2s = smem + Ly::kK2;
  const unsigned char* V1s = smem + Ly::kV1;
  const unsigned char* V2s = smem + Ly::kV2;
  const uint32_t* pvb = reinterpret_cast<const uint32_t*>(smem + Ly::kPV);
  const int nkt = (nkk + 15) >> 4;
  const int njp = (nkj + 1) >> 1;
  const int total = nkt * njp;
  int it = (wave * total) / W;
  const int it1 = ((wave + 1) * total) / W;
  const bool odd = (nkj & 1) != 0;
  constexpr uint32_t kOne2 = 0x3c003c00u;  // fp16 (1, 1)
  const mf_f32x4 zero4 = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  // BIAS: the constant part of the A operand (lane (g, r16) holds A[p = r16][K = 8g .. 8g + 7]), the
  // mask of the B halves that carry v (K in [2, 18)), and c_i as fp16 per query tile
  uint4 onehot{0u, 0u, 0u, 0u}, vmask{0u, 0u, 0u, 0u};
  uint32_t cgh[MQ];
  const unsigned char* BU = smem + Ly::kBU;
  const unsigned char* BW = smem + Ly::kBW;
  const unsigned char* BV = smem + Ly::kBV;
  if constexpr (BIAS) {
    uint32_t oh[4], vm[4];
#pragma unroll
    for (int h2 = 0; h2 < 4; ++h2) {
      uint32_t o = 0u, m = 0u;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int K = 8 * g + 2 * h2 + e;
        const bool one = K == 0 || (K >= 2 && K < 18 && r16 == K - 2);
        o |= (one ? 0x3c00u : 0u) << (16 * e);
        m |= (K >= 2 && K < 18 ? 0xffffu : 0u) << (16 * e);
      }
      oh[h2] = o;
      vm[h2] = m;
    }
    onehot = uint4{oh[0], oh[1], oh[2], oh[3]};
    vmask = uint4{vm[0], vm[1], vm[2], vm[3]};
    const float* cg = reinterpret_cast<const float*>(smem + Ly::kBG);
#pragma unroll
    for (int qt = 0; qt < MQ; ++qt)
      cgh[qt] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(cg[16 * qt + r16])));
  }
  while (it < it1) {
    const int kt = it / njp;
    int jp = it - kt * njp;
    const int jend = min(njp, jp + (it1 - it));
    it += jend - jp;
    const int k0 = kt * 16;
    // per key tile: K2 rows as the GEMM1 A operand multiplicands, the V2
    // halves of keys k0 + 4g + r as pairs (r = 0,1), (r = 2,3) per d tile,
    // and the denominator operand (1 at the valid keys)
    uint4 k2op[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      k2op[c] = *reinterpret_cast<const uint4*>(K2s + (k0 + r16) * RB + c * 64 + g * 16);
    uint32_t v2p[ND][2];
    {
      uint32_t rv[4][(ND + 1) / 2];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned char* src = V2s + (k0 + 4 * g + r) * RB + r16 * ND * 2;
        if constexpr (ND == 4) {
          const uint2 t = *reinterpret_cast<const uint2*>(src);
          rv[r][0] = t.x;
          rv[r][1] = t.y;
        } else {
          rv[r][0] = *reinterpret_cast<const uint32_t*>(src);
        }
      }
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
        v2p[dt][0] = __builtin_amdgcn_perm(rv[1][dt >> 1], rv[0][dt >> 1], sel);
        v2p[dt][1] = __builtin_amdgcn_perm(rv[3][dt >> 1], rv[2][dt >> 1], sel);
      }
    }
    uint4 bvop[MQ];
    if constexpr (BIAS) {
      // halves k0 + 8g .. k0 + 8g + 7 of the query's BV row are K = 8g .. 8g + 7 (v at k + 2)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const uint4 t = *reinterpret_cast<const uint4*>(BV + ((16 * qt + r16) * Ly::kVS + k0 + 8 * g) * 2);
        bvop[qt] = uint4{t.x & vmask.x, t.y & vmask.y, t.z & vmask.z, t.w & vmask.w};
      }
    }
    const int kvalid = nkk - (k0 + 4 * g);  // keys 4g + r valid for r < kvalid
    const uint32_t o01 = kvalid >= 2 ? kOne2 : (kvalid == 1 ? 0x00003c00u : 0u);
    const uint32_t o23 = kvalid >= 4 ? kOne2 : (kvalid == 3 ? 0x00003c00u : 0u);
    const uint4 ones_kt{o01, o23, o01, o23};
    const uint4 ones_half{o01, o23, 0u, 0u};
    const uint32_t kmask = kvalid >= 4 ? 0xfu : (kvalid <= 0 ? 0u : ((1u << kvalid) - 1u));
    int pvshift = 0, pvword = 0;
    if constexpr (HAS_PV) {
      pvword = k0 >> 5;
      pvshift = (k0 & 31) + 4 * g;
    }
    for (; jp < jend; ++jp) {
      const int j0 = 2 * jp;
      const bool last_odd = odd && jp == njp - 1;
      uint4 ka[NCH], kb[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        ka[c] = *reinterpret_cast<const uint4*>(K1s + j0 * RB + c * 64 + g * 16);
        kb[c] = *reinterpret_cast<const uint4*>(K1s + (j0 + 1) * RB + c * 64 + g * 16);
      }
      uint32_t va[(ND + 1) / 2], vb[(ND + 1) / 2];
      if constexpr (MODE != kMax) {
        if constexpr (ND == 4) {
          const uint2 ta = *reinterpret_cast<const uint2*>(V1s + j0 * RB + r16 * 8);
          const uint2 tb = *reinterpret_cast<const uint2*>(V1s + (j0 + 1) * RB + r16 * 8);
          va[0] = ta.x; va[1] = ta.y;
          vb[0] = tb.x; vb[1] = tb.y;
        } else {
          va[0] = *reinterpret_cast<const uint32_t*>(V1s + j0 * RB + r16 * 4);
          vb[0] = *reinterpret_cast<const uint32_t*>(V1s + (j0 + 1) * RB + r16 * 4);
        }
      }
      // valid keys 4g + r of rows j0 (bits_a) and j0 + 1 (bits_b)
      uint32_t bits_a = kmask, bits_b = last_odd ? 0u : kmask;
      if constexpr (HAS_PV) {
        bits_a &= pvb[j0 * Ly::kPVW + pvword] >> pvshift;
        bits_b &= pvb[(j0 + 1) * Ly::kPVW + pvword] >> pvshift;
      }
      // GEMM1 for rows j0 and j0 + 1
      uint4 wa[NCH], wb[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        wa[c] = pkmul4(ka[c], k2op[c]);
        wb[c] = pkmul4(kb[c], k2op[c]);
      }
      mf_f32x4 sa[QT], sb[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        sa[qt] = mfma(wa[0], qop[qt][0], zero4);
        sb[qt] = mfma(wb[0], qop[qt][0], zero4);
#pragma unroll
        for (int c = 1; c < NCH; ++c) {
          sa[qt] = mfma(wa[c], qop[qt][c], sa[qt]);
          sb[qt] = mfma(wb[c], qop[qt][c], sb[qt]);
        }
      }
      if constexpr (BIAS) {
        // rows j0, j0 + 1: w of the lane's pair into A (K = 1), c_i u_ij into B (K = 0), both on the g = 0
        // lanes (the padding row j0 + 1 = nkj reads zeros)
        const uint32_t w_a = *reinterpret_cast<const uint16_t*>(BW + (j0 * kCap + k0 + r16) * 2);
        const uint32_t w_b = *reinterpret_cast<const uint16_t*>(BW + ((j0 + 1) * kCap + k0 + r16) * 2);
        const uint4 ab_a{g == 0 ? (0x3c00u | (w_a << 16)) : onehot.x, onehot.y, onehot.z, onehot.w};
        const uint4 ab_b{g == 0 ? (0x3c00u | (w_b << 16)) : onehot.x, onehot.y, onehot.z, onehot.w};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const uint32_t u_a = *reinterpret_cast<const uint16_t*>(BU + (j0 * Ly::kMaxQ + 16 * qt + r16) * 2);
          const uint32_t u_b = *reinterpret_cast<const uint16_t*>(BU + ((j0 + 1) * Ly::kMaxQ + 16 * qt + r16) * 2);
          const uint4 bb_a{g == 0 ? (u_a | (cgh[qt] << 16)) : bvop[qt].x, bvop[qt].y, bvop[qt].z, bvop[qt].w};
          const uint4 bb_b{g == 0 ? (u_b | (cgh[qt] << 16)) : bvop[qt].x, bvop[qt].y, bvop[qt].z, bvop[qt].w};
          sa[qt] = mfma(ab_a, bb_a, sa[qt]);
          sb[qt] = mfma(ab_b, bb_b, sb[qt]);
        }
      }
      if constexpr (MODE == kMax) {
        // maxima of the valid logits (padded keys and rows have S = 0 and
        // must not count)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const bool ka_ok = (bits_a >> r) & 1u;
            const bool kb_ok = (bits_b >> r) & 1u;
            mloc[qt] = fmaxf(mloc[qt], ka_ok ? sa[qt][r] : -INFINITY);
            mloc[qt] = fmaxf(mloc[qt], kb_ok ? sb[qt][r] : -INFINITY);
          }
        }
      } else {
        if constexpr (MODE == kOnline) {
          // the running offset of each query (mloc, log2 units; negm = -mloc): the tile's maximum over the
          // valid logits of the query's four lane groups; when it passes the offset by more than the slack
          // the offset moves to it and the query's O and L are rescaled (2^-inf = 0 on the first move)
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            float t = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              t = fmaxf(t, ((bits_a >> r) & 1u) ? sa[qt][r] : -INFINITY);
              t = fmaxf(t, ((bits_b >> r) & 1u) ? sb[qt][r] : -INFINITY);
            }
            t = __uint_as_float(swap32_op(swap16_op(__float_as_uint(t), MaxF32{}), MaxF32{})) * sc;
            const bool up = t > mloc[qt] + kOnlineSlack;
            if (__any(up)) {
              const float mn = up ? t : mloc[qt];
              const float f = up ? __builtin_amdgcn_exp2f(mloc[qt] - mn) : 1.0f;
#pragma unroll
              for (int dt = 0; dt < ND; ++dt) O[dt][qt] *= f;
              L[qt] *= f;
              mloc[qt] = mn;
              negm[qt] = -mn;
            }
          }
        }
        // Z^T operands: d = 16 dt + r16, keys 4g + r of row j0 (halves
        // 0..3) and of row j0 + 1 (halves 4..7)
        uint4 z[ND];
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const uint32_t wa1 = va[dt >> 1], wb1 = vb[dt >> 1];
          if (dt & 1) {
            z[dt] = uint4{pkmul_splat<1>(v2p[dt][0], wa1), pkmul_splat<1>(v2p[dt][1], wa1),
                          pkmul_splat<1>(v2p[dt][0], wb1), pkmul_splat<1>(v2p[dt][1], wb1)};
          } else {
            z[dt] = uint4{pkmul_splat<0>(v2p[dt][0], wa1), pkmul_splat<0>(v2p[dt][1], wa1),
                          pkmul_splat<0>(v2p[dt][0], wb1), pkmul_splat<0>(v2p[dt][1], wb1)};
          }
        }
        uint4 pop[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float ea[4], eb[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if constexpr (MODE == kFast) {
              ea[r] = __builtin_amdgcn_exp2f(sa[qt][r]);
              eb[r] = __builtin_amdgcn_exp2f(sb[qt][r]);
            } else {
              ea[r] = __builtin_amdgcn_exp2f(fmaf(sa[qt][r], sc, negm[qt]));
              eb[r] = __builtin_amdgcn_exp2f(fmaf(sb[qt][r], sc, negm[qt]));
            }
          }
          pop[qt] = uint4{pack_h2(ea[0], ea[1]), pack_h2(ea[2], ea[3]), pack_h2(eb[0], eb[1]), pack_h2(eb[2], eb[3])};
          // two-pass mode: padded pairs have S = 0, so 2^(0 - m) may exceed
          // the fp16 range; they and the pairs pair_valid clears get P = 0
          if constexpr (HAS_PV || MODE == kSlow || MODE == kOnline) {
            pop[qt].x &= pv_mask(bits_a, 0);
            pop[qt].y &= pv_mask(bits_a, 1);
            pop[qt].z &= pv_mask(bits_b, 0);
            pop[qt].w &= pv_mask(bits_b, 1);
          }
        }
        const uint4 ones = last_odd ? ones_half : ones_kt;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
          for (int dt = 0; dt < ND; ++dt) O[dt][qt] = mfma(z[dt], pop[qt], O[dt][qt]);
          L[qt] = mfma(ones, pop[qt], L[qt]);
        }
      }
    }
  }
}

// pair_loop for the runtime tile count nqt (1 .. MQ)
template <int DP, int MODE, bool HAS_PV, bool BIAS, int MQ>
__device__ __forceinline__ void pair_loop_n(int nqt, const unsigned char* smem, int nkj, int nkk,
                                            const uint4 (&qop)[MQ][DP / 32], float (&negm)[MQ], float sc,
                                            mf_f32x4 (&O)[DP / 16][MQ], mf_f32x4 (&L)[MQ], float (&mloc)[MQ], int wave,
                                            int g, int r16) {
  static_assert(MQ == 2 || MQ == 3, "two or three query tiles");
  if (nqt == 1) pair_loop<DP, 1, MODE, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
  else if (MQ == 2 || nqt == 2) pair_loop<DP, 2, MODE, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
  else pair_loop<DP, MQ, MODE, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
}

// ---------------------------------------------------------------------------
// one unit (molecule b, head h, queries q0 .. q0 + nqg - 1 of its valid ones)
// ---------------------------------------------------------------------------
// MULTI: the unit has more than kCap keys and is taken in (j block, k block)
// pairs, with one query tile (its accumulators stay live across the block
// loop, so the group is kept small).
// Zero the output rows of the padded queries of the (b, h) pairs w, w + G,
// ... (a workgroup's share; rows of CPR 16-byte chunks, DP / 8 of them).
template <typename T, int DP, bool STR, int W>
__device__ __forceinline__ void zero_padded_share(const Params& p, const uint32_t* s_info, int w, int G) {
  constexpr int kThreads = W * 64;
  constexpr int CPR = DP / 8;
  const int N = p.N, D = p.D, H = p.H;
  const int cpr = D / 8;
  for (int bh = w; bh < p.B * H; bh += G) {
    const int b = bh / H, h = bh - b * H;
    const uint32_t info = s_info[b];
    const bool qpre = (info & kQPre) != 0;
    const int i0 = qpre ? info_nq(info) : 0;  // rows below are valid
    const uint8_t* qrow = p.qv + size_t(b) * N;
    T* orow0 = p.out ? static_cast<T*>(p.out) + (STR ? size_t(b) * p.os_b + size_t(h) * p.os_h : size_t(bh) * N * D)
                     : nullptr;
    const size_t osn = STR ? size_t(p.os_n) : size_t(D);
    for (int u = int(threadIdx.x); u < (N - i0) * CPR; u += kThreads) {
      const int i = i0 + u / CPR, cc = u % CPR;
      if (cc >= cpr || (!qpre && qrow[i] != 0)) continue;
      const size_t row = size_t(bh) * N + i;
      if (p.out) reinterpret_cast<uint4*>(orow0 + size_t(i) * osn)[cc] = uint4{0u, 0u, 0u, 0u};
      if (p.out_f32) {
        float4* o = reinterpret_cast<float4*>(p.out_f32 + row * D + cc * 8);
        o[0] = float4{0.f, 0.f, 0.f, 0.f};
        o[1] = float4{0.f, 0.f, 0.f, 0.f};
      }
      if (cc == 0 && p.lse) p.lse[row] = 0.0f;
    }
  }
}

// An element of a bias tensor as float.
__device__ __forceinline__ float bias_at(const void* t, size_t idx, int dtype) {
  if (dtype == MF_DTYPE_F32) return static_cast<const float*>(t)[idx];
  if (dtype == MF_DTYPE_BF16) return float(static_cast<const __bf16*>(t)[idx]);
  return float(static_cast<const _Float16*>(t)[idx]);
}
// fp16 bits of x, saturated to the finite range
__device__ __forceinline__ uint16_t half_bits_sat(float x) {
  return __builtin_bit_cast(uint16_t, _Float16(fminf(fmaxf(x, -65504.0f), 65504.0f)));
}

template <typename T, int DP, bool HAS_PV, bool MULTI, bool BIAS, bool STR>
__device__ __forceinline__ void unit_body(const Params& p, unsigned char* smem, int b, int h, int nk, int q0, int nqg,
                                          bool kpre, bool qpre, bool zero_share) {
  constexpr int GQ = Waves<BIAS>::kGroup;
  constexpr int QT = GQ / 16;          // query tiles held in registers
  const int nqt = (nqg + 15) >> 4;     // query tiles in use
  constexpr int kWaves = Waves<BIAS>::kCount;
  constexpr int kThreads = kWaves * 64;
  using Ly = Lay<DP, BIAS>;
  constexpr int kCap = Ly::kCap;
  constexpr int kMaxQ = Ly::kMaxQ;
  constexpr int RB = Ly::RB;
  constexpr int NCH = Shape<DP>::NCH;
  constexpr int ND = Shape<DP>::ND;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const int H = p.H, N = p.N, D = p.D;
  const int bh = b * H + h;
  const uint16_t* kidx = reinterpret_cast<const uint16_t*>(smem + Ly::kKidx);
  const uint16_t* qidx = reinterpret_cast<const uint16_t*>(smem + Ly::kQidx);
  float* colmax = reinterpret_cast<float*>(smem + Ly::kCol);
  float* mn = reinterpret_cast<float*>(smem + Ly::kMn);
  float* gmax = reinterpret_cast<float*>(smem + Ly::kG);
  int* scal = reinterpret_cast<int*>(smem + Ly::kScal);
  float* s_m = reinterpret_cast<float*>(smem + Ly::kM);
  // operand strides: the caller's (STR) or those of the contiguous [B*H, N, D] layout
  const size_t qoff = STR ? size_t(b) * p.qs_b + size_t(h) * p.qs_h : size_t(bh) * N * D;
  const size_t koff = STR ? size_t(b) * p.ks_b + size_t(h) * p.ks_h : size_t(bh) * N * D;
  const size_t qsn = STR ? size_t(p.qs_n) : size_t(D), ksn = STR ? size_t(p.ks_n) : size_t(D);
  const T* gq = static_cast<const T*>(p.q) + qoff;
  const T* gk1 = static_cast<const T*>(p.k1) + koff;
  const T* gk2 = static_cast<const T*>(p.k2) + koff;
  const T* gv1 = static_cast<const T*>(p.v1) + koff;
  const T* gv2 = static_cast<const T*>(p.v2) + koff;

  // staging map: 16-byte chunk u = tid + kThreads i of a row set is row
  // u / CPR, columns 8 cc .. 8 cc + 7 with cc = tid % CPR for every i; only
  // the rows the pair loop reads (the valid ones rounded up to 16) are staged
  constexpr int CPR = DP / 8;                        // chunks per row
  constexpr int MAXC = (kCap * CPR + kThreads - 1) / kThreads;  // chunks per thread and block
  constexpr int MAXQC = (kMaxQ * CPR + kThreads - 1) / kThreads;
  const int cc = tid % CPR;
  const int e0 = 8 * cc;
  const bool col_ok = e0 < D;
  const int nch = (nk + kCap - 1) / kCap;
  auto key_atom = [&](int rank) { return kpre ? rank : int(kidx[rank]); };
  auto round16 = [](int n) { return (n + 15) & ~15; };
  // chunk slots that hold a staged row (the rest of the MAXC are skipped by a
  // scalar branch, not issued under an empty exec mask): all of them for key
  // blocks, else those of the valid rows rounded up to 16
  const int nI = MULTI ? MAXC : __builtin_amdgcn_readfirstlane((round16(nk) * CPR + kThreads - 1) / kThreads);
  // rows [row0, row0 + nrows) of the compacted keys; rows up to the next
  // multiple of 16 read as zero.  The atom indices of a block's slots are
  // read once (rows clamped into the block) for its key and value sets, so
  // the loads are not each preceded by an index read and its wait.
  auto slot_atoms = [&](int row0, int nrows, int (&atom)[MAXC]) {
    const int rlast = max(nrows - 1, 0);
#pragma unroll
    for (int i = 0; i < MAXC; ++i)
      atom[i] = nrows > 0 ? key_atom(row0 + min((tid + kThreads * i) / CPR, rlast)) : 0;
  };
  auto load_set = [&](const T* base, const int (&atom)[MAXC], int nrows, uint4 (&arr)[MAXC]) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int row = (tid + kThreads * i) / CPR;
      arr[i] = uint4{0u, 0u, 0u, 0u};
      if (i < nI && row < nrows && col_ok) arr[i] = *reinterpret_cast<const uint4*>(base + size_t(atom[i]) * ksn + e0);
    }
  };
  uint4 rk1[MAXC], rk2[MAXC], rv1[MAXC], rv2[MAXC], rq[MAXQC];
  // every slot without a branch, for the maxima only: rows clamped into the
  // block repeat a valid row (maxima unchanged), columns past D read column
  // 0 and are masked in acc_max.  (Conditional loads joined with zeros would
  // make the compiler wait for each load in its own branch.)
  auto load_set_all = [&](const T* base, const int (&atom)[MAXC], uint4 (&arr)[MAXC]) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) arr[i] = *reinterpret_cast<const uint4*>(base + size_t(atom[i]) * ksn + (col_ok ? e0 : 0));
  };
  auto load_block = [&](int jc, int kc) {
    const int j0 = jc * kCap, k0 = kc * kCap;
    const int nkj = min(kCap, nk - j0), nkk = min(kCap, nk - k0);
    int aj[MAXC], ak[MAXC];
    slot_atoms(j0, nkj, aj);
    if (kc == jc) {
#pragma unroll
      for (int i = 0; i < MAXC; ++i) ak[i] = aj[i];
    } else {
      slot_atoms(k0, nkk, ak);
    }
    load_set(gk1, aj, nkj, rk1);
    load_set(gv1, aj, nkj, rv1);
    load_set(gk2, ak, nkk, rk2);
    load_set(gv2, ak, nkk, rv2);
  };

  // ---- phase A: maxima -> scale exponents -------------------------------
  // magnitudes as 16-bit patterns (|x| of bf16 / fp16 orders like its bits
  // with the sign cleared), two per dword, reduced with v_pk_max_u16
  uint32_t c1[4], c2[4];  // column maxima of |K1|, |K2| for columns e0 .. e0 + 7
  uint32_t gv = 0u, gqm = 0u;  // |V1| (low half) and |V2| (high half) maxima; |q| maxima
#pragma unroll
  for (int e = 0; e < 4; ++e) c1[e] = c2[e] = 0u;
  const uint32_t cmask = col_ok ? 0x7fff7fffu : 0u;  // magnitude bits; nothing for columns past D
  auto acc_max = [&]() {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      if (i >= nI) break;
      const uint32_t a1[4] = {rk1[i].x, rk1[i].y, rk1[i].z, rk1[i].w};
      const uint32_t a2[4] = {rk2[i].x, rk2[i].y, rk2[i].z, rk2[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c1[e] = pk_max_u16(c1[e], a1[e] & cmask);
        c2[e] = pk_max_u16(c2[e], a2[e] & cmask);
      }
      const uint32_t m1 = pk_max_u16(pk_max_u16(rv1[i].x, rv1[i].y), pk_max_u16(rv1[i].z, rv1[i].w)) & cmask;
      const uint32_t m2 = pk_max_u16(pk_max_u16(rv2[i].x, rv2[i].y), pk_max_u16(rv2[i].z, rv2[i].w)) & cmask;
      // low half: |V1|, high half: |V2|
      gv = pk_max_u16(gv, __builtin_amdgcn_perm(m2, m1, 0x07060302u));
      gv = pk_max_u16(gv, __builtin_amdgcn_perm(m2, m1, 0x05040100u));
    }
  };
  {
    // query rows of the group (rows >= nqg read as zero; indices first, as
    // in load_set)
    const int qlast = max(nqg - 1, 0);
    int qatom[MAXQC];
#pragma unroll
    for (int i = 0; i < MAXQC; ++i) {
      const int r = q0 + min((tid + kThreads * i) / CPR, qlast);
      qatom[i] = nqg > 0 ? (qpre ? r : int(qidx[r])) : 0;
    }
#pragma unroll
    for (int i = 0; i < MAXQC; ++i) {
      const int row = (tid + kThreads * i) / CPR;
      rq[i] = uint4{0u, 0u, 0u, 0u};
      if (row < nqg && col_ok) rq[i] = *reinterpret_cast<const uint4*>(gq + size_t(qatom[i]) * qsn + e0);
    }
  }
  // ---- factorized bias (BIAS): c_i, then the fp16 operands of a block ------
  float* cgf = reinterpret_cast<float*>(smem + Ly::kBG);
  float* bmax = reinterpret_cast<float*>(smem + Ly::kBMax);  // max |u|, |v|, |w| of the unit's staged values
  // (j block, k block): BU[j][i] = c_i u_ij, BW[j][k] = w_jk, BV[i][k + 2] = c_i v_ik over the staged rows,
  // zero past the valid keys and queries
  auto stage_bias = [&](int jc, int kc, int cE) {
    uint16_t* BU = reinterpret_cast<uint16_t*>(smem + Ly::kBU);
    uint16_t* BW = reinterpret_cast<uint16_t*>(smem + Ly::kBW);
    uint16_t* BV = reinterpret_cast<uint16_t*>(smem + Ly::kBV);
    const int j0 = jc * kCap, k0 = kc * kCap;
    const int nkj = min(kCap, nk - j0), nkk = min(kCap, nk - k0);
    const int rj = round16(nkj), rk = round16(nkk);
    const int dt = p.bias_dtype;
    float mx[3] = {0.0f, 0.0f, 0.0f};  // max |u|, |v|, |w| of the staged values
    // Each set is taken a row per wave (rows wave, wave + kWaves, ...) with the lanes along the
    // columns (lane, lane + 64), so a wave's loads of a row are one coalesced run; kRB rows of a
    // wave are loaded before any is converted and stored.  Rows and columns past the valid
    // queries / keys are stored as zero.
    //   set 0 (U): rows = queries qi < kMaxQ, columns j < rj:  BU[j][qi]     = c_qi u[qa][ka(j0 + j)]
    //   set 1 (V): rows = queries qi,          columns k < rk:  BV[qi][k + 2] = c_qi v[qa][ka(k0 + k)]
    //   set 2 (W): rows j < rj,                columns k < rk:  BW[j][k]      = w[ka(j0 + j)][ka(k0 + k)]
    // Batches of kRB rows per wave: the U and V rows of a batch, its gates and, in the first batch, the
    // first W rows are loaded before anything is stored (GQ / (kWaves kRB) round trips for U and V);
    // c_i = log2(e) 2^cE gate_i is formed in registers (and stored to BG).
    constexpr int kRB = 4;
    static_assert(GQ % (kWaves * kRB) == 0, "whole batches of query rows");
    auto set_shape = [&](auto set_tag, int& R, int& C, int& rvalid, int& cvalid, int& cbase, const void*& src) {
      constexpr int SET = decltype(set_tag)::value;
      R = SET == 2 ? rj : GQ;
      C = SET == 0 ? rj : rk;
      rvalid = SET == 2 ? nkj : nqg;
      cvalid = SET == 0 ? nkj : nkk;
      cbase = SET == 0 ? j0 : k0;
      src = SET == 0 ? p.bu : (SET == 1 ? p.bv : p.bw);
    };
    // Loads without branches: a lane's two column atoms are found once, each row's atom once
    // (wave-uniform), out-of-range rows and columns read a clamped valid element (zeroed when
    // stored, so no use follows a load and a wave's loads of a batch are in flight together),
    // and the element width is one uniform choice for the whole batch.
    auto load_rows = [&](auto set_tag, int r0, uint32_t (&val)[kRB][2]) {
      constexpr int SET = decltype(set_tag)::value;
      int R, C, rvalid, cvalid, cbase;
      const void* src;
      set_shape(set_tag, R, C, rvalid, cvalid, cbase, src);
#pragma unroll
      for (int t = 0; t < kRB; ++t) val[t][0] = val[t][1] = 0u;
      if (rvalid <= 0 || cvalid <= 0) return;
      const bool two = kCap > 64 && C > 64;  // a second column per lane (wave-uniform)
      int ca[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) ca[s] = key_atom(cbase + min(lane + 64 * s, cvalid - 1));
      int ra[kRB];  // row atoms, all found before any load is issued
#pragma unroll
      for (int t = 0; t < kRB; ++t) {
        const int rc = min(r0 + kWaves * t, rvalid - 1);
        ra[t] = SET == 2 ? key_atom(j0 + rc) : (qpre ? q0 + rc : int(qidx[q0 + rc]));
      }
      auto batch = [&](auto wide_tag) {
        constexpr bool WIDE = decltype(wide_tag)::value;
#pragma unroll
        for (int t = 0; t < kRB; ++t) {
          const size_t rowbase = (size_t(bh) * N + ra[t]) * N;
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            if (s == 1 && !two) continue;  // wave-uniform
            if constexpr (WIDE) val[t][s] = static_cast<const uint32_t*>(src)[rowbase + ca[s]];
            else val[t][s] = static_cast<const uint16_t*>(src)[rowbase + ca[s]];
          }
        }
      };
      if (dt == MF_DTYPE_F32) batch(std::true_type{});
      else batch(std::false_type{});
    };
    auto store_rows = [&](auto set_tag, int r0, const uint32_t (&val)[kRB][2], const float (&crow)[kRB]) {
      constexpr int SET = decltype(set_tag)::value;
      int R, C, rvalid, cvalid, cbase;
      const void* src;
      set_shape(set_tag, R, C, rvalid, cvalid, cbase, src);
#pragma unroll
      for (int t = 0; t < kRB; ++t) {
        const int r = r0 + kWaves * t;
        if (r >= R) break;  // wave-uniform
#pragma unroll
        for (int s = 0; s < (kCap > 64 ? 2 : 1); ++s) {
          const int c = lane + 64 * s;
          if (c >= C) continue;
          const uint32_t raw = val[t][s];
          const float x = !(r < rvalid && c < cvalid) ? 0.0f
                          : dt == MF_DTYPE_F32         ? __uint_as_float(raw)
                          : dt == MF_DTYPE_BF16        ? __uint_as_float(raw << 16)
                                                       : float(__builtin_bit_cast(_Float16, uint16_t(raw)));
          mx[SET] = fmaxf(mx[SET], fabsf(x));
          if constexpr (SET == 0) BU[c * kMaxQ + r] = half_bits_sat(crow[t] * x);
          else if constexpr (SET == 1) BV[r * Ly::kVS + c + 2] = half_bits_sat(crow[t] * x);
          else BW[r * kCap + c] = half_bits_sat(x);
        }
      }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    const float kNoRow[kRB] = {};
#pragma unroll 1
    for (int qb = 0; qb < GQ / (kWaves * kRB); ++qb) {
      const int r0 = wave + kWaves * kRB * qb;
      uint32_t vu[kRB][2], vv[kRB][2], vw[kRB][2];
      float crow[kRB];
      load_rows(S0{}, r0, vu);
      load_rows(S1{}, r0, vv);
      if (qb == 0) load_rows(S2{}, r0, vw);
      // the gates of query rows wave + kWaves t: all loaded (one uniform width) before any is used
      uint32_t graw[kRB];
      int gidx[kRB];
#pragma unroll
      for (int t = 0; t < kRB; ++t) {
        const int rc = min(r0 + kWaves * t, max(nqg - 1, 0));
        gidx[t] = qpre ? q0 + rc : int(qidx[q0 + rc]);
      }
      if (dt == MF_DTYPE_F32) {
#pragma unroll
        for (int t = 0; t < kRB; ++t) graw[t] = static_cast<const uint32_t*>(p.bg)[size_t(bh) * N + gidx[t]];
      } else {
#pragma unroll
        for (int t = 0; t < kRB; ++t) graw[t] = static_cast<const uint16_t*>(p.bg)[size_t(bh) * N + gidx[t]];
      }
#pragma unroll
      for (int t = 0; t < kRB; ++t) {
        const int r = r0 + kWaves * t;
        const float gte = dt == MF_DTYPE_F32 ? __uint_as_float(graw[t])
                          : dt == MF_DTYPE_BF16 ? __uint_as_float(graw[t] << 16)
                                                : float(__builtin_bit_cast(_Float16, uint16_t(graw[t])));
        crow[t] = r < nqg ? ldexpf(gte * kLog2e, cE) : 0.0f;
      }
      store_rows(S0{}, r0, vu, crow);
      store_rows(S1{}, r0, vv, crow);
      if (qb == 0) store_rows(S2{}, r0, vw, kNoRow);
      if (lane == 0) {
#pragma unroll
        for (int t = 0; t < kRB; ++t) cgf[r0 + kWaves * t] = crow[t];
      }
    }
    // W rows past the first batch (more than kWaves kRB staged keys)
    for (int r0 = wave + kWaves * kRB; r0 < rj; r0 += kWaves * kRB) {
      uint32_t vw[kRB][2];
      load_rows(S2{}, r0, vw);
      store_rows(S2{}, r0, vw, kNoRow);
    }
    // maxima over the wave, into this wave's slots (float order equals bit order for magnitudes)
#pragma unroll
    for (int e = 0; e < 3; ++e) {
      const uint32_t m = group_reduce<64>(__float_as_uint(mx[e]), MaxF32{});
      if (lane == 0) bmax[wave * 3 + e] = __uint_as_float(m);
    }
  };
  ClaimState* cl = reinterpret_cast<ClaimState*>(smem + Ly::kClaim);
  // K rows: row-major fp16 scaled by 2^sc_exp
  auto store_k = [&](unsigned char* dst, const uint4& v, int row, int sc_exp) {
    float f[8];
    uint32_t w[4];
    unpack8<T>(v, f);
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack_h2(ldexpf(f[2 * e], sc_exp), ldexpf(f[2 * e + 1], sc_exp));
    *reinterpret_cast<uint4*>(dst + row * RB + e0 * 2) = uint4{w[0], w[1], w[2], w[3]};
  };
  // V rows: [row][r16][dt]: column d = 16 dt + r16 at half r16 ND + dt
  auto store_v = [&](unsigned char* dst, const uint4& v, int row, int sc_exp) {
    float f[8];
    unpack8<T>(v, f);
    unsigned char* a = dst + row * RB + ((8 * (cc & 1)) * ND + (cc >> 1)) * 2;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      *reinterpret_cast<_Float16*>(a + e * ND * 2) = _Float16(ldexpf(f[e], sc_exp));
  };
  // bits of pair_valid for rows j of the j block and keys k of the k block
  auto stage_pv = [&](int jc, int kc) {
    uint32_t* pvb = reinterpret_cast<uint32_t*>(smem + Ly::kPV);
    const uint8_t* gpv = p.pv + size_t(b) * N * N;
    const int j0 = jc * kCap, k0 = kc * kCap;
    const int nkj = min(kCap, nk - j0), nkk = min(kCap, nk - k0);
    // a word's bytes are loaded 16 at a time without branches (columns past the block read its last key,
    // and are masked afterwards), so each 16 loads are in flight together
    for (int u = tid; u < kCap * Ly::kPVW; u += kThreads) {
      const int jl = u / Ly::kPVW, wd = u % Ly::kPVW;
      uint32_t bits = 0;
      if (jl < nkj && nkk > 0) {
        const uint8_t* prow = gpv + size_t(key_atom(j0 + jl)) * N;
#pragma unroll 1
        for (int h = 0; h < 32; h += 16) {
          uint8_t v[16];
#pragma unroll
          for (int t = 0; t < 16; ++t) v[t] = prow[key_atom(k0 + min(wd * 32 + h + t, nkk - 1))];
#pragma unroll
          for (int t = 0; t < 16; ++t) bits |= (wd * 32 + h + t < nkk && v[t] != 0) ? 1u << (h + t) : 0u;
        }
      }
      pvb[u] = bits;
    }
  };
  // GUESS: the unit is staged with unit scales (K, V as they are, Q as q log2(e)) straight from the loads,
  // before the maxima are known; after the one barrier every wave checks the maxima against the range in
  // which unit scales give the results of the normalised scales (every staged value, product and P stays
  // a normal fp16 number, and fp16 rounding is scale-invariant there) and against a looser |S| bound,
  // max_i ||q'_i||_1 max|K1| max|K2|.  A unit outside it is staged again the normalised way.
  constexpr bool GUESS = !MULTI && !BIAS;
  float ql1 = 0.0f;  // GUESS: the largest ||q'_i||_1 of this wave's query rows
  if constexpr (!MULTI) {
    load_block(0, 0);
    // without the bias: the pair-valid bits of the unit's one block, while the key rows are in flight (with
    // the bias they are staged with the block, after the bias: staged here, their waits held up the bias
    // loads)
    if constexpr (HAS_PV && !BIAS) stage_pv(0, 0);
    // the workgroup's share of padded query rows, stored while the loads are
    // in flight (first unit only)
    if (zero_share) zero_padded_share<T, DP, STR, Waves<BIAS>::kCount>(p, reinterpret_cast<const uint32_t*>(smem + Ly::kInfo), blockIdx.x, gridDim.x);
    // the bias operands, loaded while the key rows are in flight (query scale exponent E = 0 assumed)
    if constexpr (BIAS) stage_bias(0, 0, 0);
    if constexpr (GUESS) {
      const int rj = round16(nk);
#pragma unroll
      for (int i = 0; i < MAXC; ++i) {
        if (i >= nI) break;
        const int row = (tid + kThreads * i) / CPR;
        if (row < rj) {
          store_k(smem + Ly::kK1, rk1[i], row, 0);
          store_v(smem + Ly::kV1, rv1[i], row, 0);
          store_k(smem + Ly::kK2, rk2[i], row, 0);
          store_v(smem + Ly::kV2, rv2[i], row, 0);
        }
      }
      unsigned char* Qs = smem + Ly::kQ;
#pragma unroll
      for (int i = 0; i < MAXQC; ++i) {
        const int row = (tid + kThreads * i) / CPR;
        float f[8];
        unpack8<T>(rq[i], f);
        float l1 = 0.0f;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          f[e] *= kLog2e;
          l1 += fabsf(f[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack_h2(f[2 * e], f[2 * e + 1]);
        if (row < kMaxQ) *reinterpret_cast<uint4*>(Qs + row * RB + e0 * 2) = uint4{w[0], w[1], w[2], w[3]};
        l1 = __uint_as_float(group_reduce<CPR>(__float_as_uint(l1), AddF32{}));
        ql1 = fmaxf(ql1, row < nqg ? l1 : 0.0f);
      }
    }
    acc_max();
  } else {
    if (zero_share) zero_padded_share<T, DP, STR, Waves<BIAS>::kCount>(p, reinterpret_cast<const uint32_t*>(smem + Ly::kInfo), blockIdx.x, gridDim.x);
    for (int rc = 0; rc < nch; ++rc) {
      int a[MAXC];
      slot_atoms(rc * kCap, min(kCap, nk - rc * kCap), a);
      load_set_all(gk1, a, rk1);
      load_set_all(gv1, a, rv1);
      load_set_all(gk2, a, rk2);
      load_set_all(gv2, a, rv2);
      acc_max();
    }
  }
#pragma unroll
  for (int i = 0; i < MAXQC; ++i)
    gqm = pk_max_u16(gqm, pk_max_u16(pk_max_u16(rq[i].x, rq[i].y), pk_max_u16(rq[i].z, rq[i].w)) & 0x7fff7fffu);
  {
    // column maxima over the lanes that share cc, then per wave to LDS
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      c1[e] = stride_reduce<CPR>(c1[e], PkMaxU16{});
      c2[e] = stride_reduce<CPR>(c2[e], PkMaxU16{});
    }
    gv = group_reduce<64>(gv, PkMaxU16{});
    gqm = group_reduce<64>(gqm, PkMaxU16{});
    if constexpr (GUESS) ql1 = __uint_as_float(group_reduce<64>(__float_as_uint(ql1), MaxF32{}));
    uint32_t* colw = reinterpret_cast<uint32_t*>(colmax);  // [kWaves][2][DP / 2] packed pairs
    if (lane < CPR) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        colw[(wave * 2 + 0) * (DP / 2) + 4 * lane + e] = c1[e];
        colw[(wave * 2 + 1) * (DP / 2) + 4 * lane + e] = c2[e];
      }
    }
    if (lane == 0) {
      uint32_t* gw = reinterpret_cast<uint32_t*>(gmax);
      gw[wave * 4 + 0] = gv;
      gw[wave * 4 + 1] = gqm;
      gw[wave * 4 + 2] = __float_as_uint(ql1);
    }
  }
  __syncthreads();
  // GUESS: every wave combines the partials (the same values in every wave, so every wave takes the same
  // branch) and keeps the unit-scale staging when it is valid
  bool staged = false;
  if constexpr (GUESS) {
    const uint32_t* colw = reinterpret_cast<const uint32_t*>(colmax);
    const uint32_t* gw = reinterpret_cast<const uint32_t*>(gmax);
    float m1 = 0.0f, m2 = 0.0f;
    if (lane < DP) {
      uint32_t w1 = 0u, w2 = 0u;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        w1 = max(w1, (colw[(w * 2 + 0) * (DP / 2) + lane / 2] >> (16 * (lane & 1))) & 0xffffu);
        w2 = max(w2, (colw[(w * 2 + 1) * (DP / 2) + lane / 2] >> (16 * (lane & 1))) & 0xffffu);
      }
      m1 = mag_to_float<T>(w1);
      m2 = mag_to_float<T>(w2);
    }
    const float a1 = __uint_as_float(group_reduce<64>(__float_as_uint(m1), MaxF32{}));
    const float a2 = __uint_as_float(group_reduce<64>(__float_as_uint(m2), MaxF32{}));
    uint32_t v = 0u, qm = 0u;
    float qn = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      v = pk_max_u16(v, gw[w * 4 + 0]);
      qm = pk_max_u16(qm, gw[w * 4 + 1]);
      qn = fmaxf(qn, __uint_as_float(gw[w * 4 + 2]));
    }
    const float b1 = mag_to_float<T>(v & 0xffffu), b2 = mag_to_float<T>(v >> 16);
    const float bq = fmaxf(mag_to_float<T>(qm & 0xffffu), mag_to_float<T>(qm >> 16));
    // unit scale is the normalised one up to a factor 2^s, |s| <= 3, for every operand
    auto in_range = [](float a) { return a == 0.0f || (a >= 0.125f && a < 16.0f); };
    staged = in_range(a1) && in_range(a2) && in_range(b1) && in_range(b2) && bq * kLog2e < kQLimit &&
             qn * (a1 * a2) <= kBoundLimit;
  }
  if (!staged && wave == 0) {
    const uint32_t* colw = reinterpret_cast<const uint32_t*>(colmax);
    float m1 = 0.0f, m2 = 0.0f;
    if (lane < DP) {
      uint32_t w1 = 0u, w2 = 0u;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        w1 = max(w1, (colw[(w * 2 + 0) * (DP / 2) + lane / 2] >> (16 * (lane & 1))) & 0xffffu);
        w2 = max(w2, (colw[(w * 2 + 1) * (DP / 2) + lane / 2] >> (16 * (lane & 1))) & 0xffffu);
      }
      m1 = mag_to_float<T>(w1);
      m2 = mag_to_float<T>(w2);
      mn[lane] = m1 * m2;
    }
    const float a1 = __uint_as_float(group_reduce<64>(__float_as_uint(m1), MaxF32{}));
    const float a2 = __uint_as_float(group_reduce<64>(__float_as_uint(m2), MaxF32{}));
    if (lane == 0) {
      const uint32_t* gw = reinterpret_cast<const uint32_t*>(gmax);
      uint32_t v = 0u, qm = 0u;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        v = pk_max_u16(v, gw[w * 4 + 0]);
        qm = pk_max_u16(qm, gw[w * 4 + 1]);
      }
      const float b1 = mag_to_float<T>(v & 0xffffu), b2 = mag_to_float<T>(v >> 16);
      const float bq = fmaxf(mag_to_float<T>(qm & 0xffffu), mag_to_float<T>(qm >> 16));
      const int s1 = norm_exp(a1), s2 = norm_exp(a2);
      const int t1 = norm_exp(b1), t2 = norm_exp(b2);
      const float cq = bq * kLog2e;
      int sq = -(s1 + s2);
      int E = 0;
      if (!(ldexpf(cq, sq) < kQLimit)) {
        sq = norm_exp(cq);
        E = s1 + s2 + sq;
      }
      scal[0] = s1;
      scal[1] = s2;
      scal[2] = t1;
      scal[3] = t2;
      scal[4] = sq;
      scal[5] = E;
      scal[6] = E != 0 ? 1 : 0;  // two-pass flag (queries add theirs)
      scal[7] = E != 0 ? 1 : 0;  // no shifted one-pass (queries add theirs)
    }
  }
  if (!staged) __syncthreads();
  const int s1 = staged ? 0 : scal[0], s2 = staged ? 0 : scal[1], t1 = staged ? 0 : scal[2];
  const int t2 = staged ? 0 : scal[3], sq = staged ? 0 : scal[4], E = staged ? 0 : scal[5];

  if constexpr (BIAS) {
    if constexpr (!MULTI) {
      // staged with the key rows assuming E = 0; a query scale of its own (E != 0, rare) restages
      if (E != 0) {
        __syncthreads();
        stage_bias(0, 0, E);
        __syncthreads();
      }
    } else {
      if (tid == 0) scal[6] = 1;  // blocks stage their bias one pair at a time: exact offsets (online pass)
    }
  }
  float bias_mag = 0.0f;
  if constexpr (BIAS) {
    float m3[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
#pragma unroll
      for (int e = 0; e < 3; ++e) m3[e] = fmaxf(m3[e], bmax[w * 3 + e]);
    bias_mag = m3[0] + m3[1] + m3[2];
  }

  // ---- phase B: query rows, bounds ---------------------------------------
  if (!staged) {
    unsigned char* Qs = smem + Ly::kQ;
    const float4 mlo = *reinterpret_cast<const float4*>(mn + e0);
    const float4 mhi = *reinterpret_cast<const float4*>(mn + e0 + 4);
    const float mm[8] = {mlo.x, mlo.y, mlo.z, mlo.w, mhi.x, mhi.y, mhi.z, mhi.w};
#pragma unroll
    for (int i = 0; i < MAXQC; ++i) {
      const int row = (tid + kThreads * i) / CPR;
      float f[8];
      unpack8<T>(rq[i], f);
      float ub = 0.0f;
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float qq = f[e] * kLog2e;
        ub = fmaf(fabsf(qq), mm[e], ub);
        f[e] = ldexpf(qq, sq);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = pack_h2(f[2 * e], f[2 * e + 1]);
      if (row < 16 * QT) *reinterpret_cast<uint4*>(Qs + row * RB + e0 * 2) = uint4{w[0], w[1], w[2], w[3]};
      // |S| bound of the row: the CPR lanes of a row are consecutive
      ub = __uint_as_float(group_reduce<CPR>(__float_as_uint(ub), AddF32{}));
      if constexpr (BIAS) {
        if (row < nqg) ub += fabsf(cgf[row]) * bias_mag;
      }
      if (row < nqg && cc == 0 && !(ub <= kBoundLimit)) atomicOr(&scal[6], 1);
      if (row < nqg && cc == 0 && !(ub <= kShiftMax)) atomicOr(&scal[7], 1);
      // the query's offset in the shifted one-pass mode (0 for padded rows)
      if (cc == 0 && row < 16 * QT) s_m[row] = row < nqg ? fmaxf(ub - kShiftTop, 0.0f) : 0.0f;
    }
  }

  // ---- staging of one (j block, k block) ----------------------------------
  auto store_block = [&](int jc, int kc) {
    unsigned char* K1s = smem + Ly::kK1;
    unsigned char* K2s = smem + Ly::kK2;
    unsigned char* V1s = smem + Ly::kV1;
    unsigned char* V2s = smem + Ly::kV2;
    const int nkj = min(kCap, nk - jc * kCap), nkk = min(kCap, nk - kc * kCap);
    const int rj = round16(nkj), rk = round16(nkk);
    if constexpr (!MULTI) {
      // the rows loaded in phase A
#pragma unroll
      for (int i = 0; i < MAXC; ++i) {
        if (i >= nI) break;
        const int row = (tid + kThreads * i) / CPR;
        if (row < rj) {
          store_k(K1s, rk1[i], row, s1);
          store_v(V1s, rv1[i], row, t1);
        }
        if (row < rk) {
          store_k(K2s, rk2[i], row, s2);
          store_v(V2s, rv2[i], row, t2);
        }
      }
    } else {
      // larger molecules: one tensor at a time, so that few registers are
      // live next to the accumulators
      const int j0 = jc * kCap, k0 = kc * kCap;
      uint4 t[MAXC];
      int aj[MAXC], ak[MAXC];
      slot_atoms(j0, nkj, aj);
      slot_atoms(k0, nkk, ak);
      load_set(gk1, aj, nkj, t);
#pragma unroll
      for (int i = 0; i < MAXC; ++i)
        if ((tid + kThreads * i) / CPR < rj) store_k(K1s, t[i], (tid + kThreads * i) / CPR, s1);
      load_set(gv1, aj, nkj, t);
#pragma unroll
      for (int i = 0; i < MAXC; ++i)
        if ((tid + kThreads * i) / CPR < rj) store_v(V1s, t[i], (tid + kThreads * i) / CPR, t1);
      load_set(gk2, ak, nkk, t);
#pragma unroll
      for (int i = 0; i < MAXC; ++i)
        if ((tid + kThreads * i) / CPR < rk) store_k(K2s, t[i], (tid + kThreads * i) / CPR, s2);
      load_set(gv2, ak, nkk, t);
#pragma unroll
      for (int i = 0; i < MAXC; ++i)
        if ((tid + kThreads * i) / CPR < rk) store_v(V2s, t[i], (tid + kThreads * i) / CPR, t2);
    }
    if constexpr (BIAS && MULTI) stage_bias(jc, kc, E);
    if constexpr (HAS_PV && (MULTI || BIAS)) stage_pv(jc, kc);
  };

  // ---- phase C: pair loop -------------------------------------------------
  uint4 qop[QT][NCH];
  mf_f32x4 O[ND][QT], L[QT];
  float mloc[QT], negm[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    L[qt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
    mloc[qt] = -INFINITY;
    negm[qt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) O[dt][qt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float sc = ldexpf(1.0f, -E);
  auto load_qop = [&]() {
    const unsigned char* Qs = smem + Ly::kQ;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int cc = 0; cc < NCH; ++cc)
        if (qt < nqt)
        qop[qt][cc] = *reinterpret_cast<const uint4*>(Qs + (16 * qt + r16) * RB + cc * 64 + g * 16);
  };
  // per-query maxima of the two-pass mode: reduce the waves' partial maxima
  auto finish_max = [&]() {
    float* redm = colmax;  // [kWaves][kMaxQ]
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float m = __uint_as_float(swap32_op(swap16_op(__float_as_uint(mloc[qt]), MaxF32{}), MaxF32{}));
      if (g == 0) redm[wave * kMaxQ + 16 * qt + r16] = m;
    }
    __syncthreads();
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float m = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) m = fmaxf(m, redm[w * kMaxQ + 16 * qt + r16]);
      m = m == -INFINITY ? 0.0f : m * sc;  // log2 units
      negm[qt] = -m;
      if (wave == 0 && g == 0) s_m[16 * qt + r16] = m;
    }
  };
  // after a kOnline pass: every wave moves its partial O and L to the queries' common offset, the largest of
  // the waves' running offsets, which becomes the lse offset
  auto combine_online = [&]() {
    float* redm = colmax;  // [kWaves][kMaxQ]
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
      if (g == 0) redm[wave * kMaxQ + 16 * qt + r16] = mloc[qt];
    __syncthreads();
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float m = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) m = fmaxf(m, redm[w * kMaxQ + 16 * qt + r16]);
      const float f = mloc[qt] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mloc[qt] - m);
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) O[dt][qt] *= f;
      L[qt] *= f;
      if (wave == 0 && g == 0) s_m[16 * qt + r16] = m == -INFINITY ? 0.0f : m;
    }
  };
  auto start_online = [&]() {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      mloc[qt] = -INFINITY;
      negm[qt] = INFINITY;
    }
  };
  bool slow = false;
  if (!MULTI && nch == 1) {
    if (!staged) {
      store_block(0, 0);
      __syncthreads();
      slow = scal[6] != 0;
    }
    load_qop();
    if (!slow) {
      pair_loop_n<DP, kFast, HAS_PV, BIAS>(nqt, smem, nk, nk, qop, negm, sc, O, L, mloc, wave, g, r16);
    } else {
      bool exact = staged || scal[7] != 0;
      if (!exact) {
        // shifted one pass, then every wave sums the waves' denominators of all queries (the same
        // values in every wave, so every wave takes the same branch)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) negm[qt] = -s_m[16 * qt + r16];
        pair_loop_n<DP, kSlow, HAS_PV, BIAS>(nqt, smem, nk, nk, qop, negm, sc, O, L, mloc, wave, g, r16);
        float* redm = colmax;  // [kWaves][kMaxQ]
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          if (g == 0) redm[wave * kMaxQ + 16 * qt + r16] = L[qt][0];
        __syncthreads();
        bool low = false;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float l = 0.0f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w) l += redm[w * kMaxQ + 16 * qt + r16];
          const int q = 16 * qt + r16;
          low |= q < nqg && s_m[q] > 0.0f && !(l >= kMinMass);
        }
        exact = __any(low);
        if (exact) {
          __syncthreads();  // every wave has read the denominators before the exact way reuses the area
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            L[qt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
            mloc[qt] = -INFINITY;
            negm[qt] = 0.0f;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) O[dt][qt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
      if (exact && !BIAS) {
        pair_loop_n<DP, kMax, HAS_PV, BIAS>(nqt, smem, nk, nk, qop, negm, sc, O, L, mloc, wave, g, r16);
        finish_max();
        pair_loop_n<DP, kSlow, HAS_PV, BIAS>(nqt, smem, nk, nk, qop, negm, sc, O, L, mloc, wave, g, r16);
      } else if (exact) {
        // (the bias instantiations) one pass with running offsets (mloc = -inf, negm = +inf until a query's
        // first valid logit), then the waves' common offsets
        start_online();
        pair_loop_n<DP, kOnline, HAS_PV, BIAS>(nqt, smem, nk, nk, qop, negm, sc, O, L, mloc, wave, g, r16);
        combine_online();
      }
    }
  } else if (MULTI && nch > 1 && BIAS) {
    // the bias key-block path (always exact offsets): one pass over the block pairs with running offsets
    __syncthreads();
    slow = true;
    load_qop();
    start_online();
    for (int jc = 0; jc < nch; ++jc) {
      for (int kc = 0; kc < nch; ++kc) {
        store_block(jc, kc);
        __syncthreads();
        const int nkj = min(kCap, nk - jc * kCap), nkk = min(kCap, nk - kc * kCap);
        pair_loop<DP, 1, kOnline, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
        __syncthreads();
      }
    }
    combine_online();
  } else if (MULTI && nch > 1) {
    __syncthreads();
    slow = scal[6] != 0;
    load_qop();
    for (int pass = slow ? 0 : 1; pass < 2; ++pass) {
      for (int jc = 0; jc < nch; ++jc) {
        for (int kc = 0; kc < nch; ++kc) {
          store_block(jc, kc);
          __syncthreads();
          const int nkj = min(kCap, nk - jc * kCap), nkk = min(kCap, nk - kc * kCap);
          if (pass == 0)
            pair_loop<DP, 1, kMax, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
          else if (slow)
            pair_loop<DP, 1, kSlow, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
          else
            pair_loop<DP, 1, kFast, HAS_PV, BIAS>(smem, nkj, nkk, qop, negm, sc, O, L, mloc, wave, g, r16);
          __syncthreads();
        }
      }
      if (pass == 0) finish_max();
    }
  }

  // the next position, claimed now: the atomic's round trip overlaps the
  // output of this unit
  const bool claiming = tid == 0;
  unsigned int ticket = 0u;
  if (claiming) ticket = atomicAdd(p.counter, 1u);

  // ---- phase D: reduce the waves' partials, normalise, write ---------------
  __syncthreads();  // every wave is done with K/V (the reduction area aliases them)
  float* red = reinterpret_cast<float*>(smem + Ly::kRed);
  float* redl = reinterpret_cast<float*>(smem + Ly::kRedL);
  // kRedWaves slots: with 8 waves, wave w + 4 hands its partials to wave w first
  const int slot = wave & (kRedWaves - 1);
  auto put_partials = [&]() {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      if (qt >= nqt) continue;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
        *reinterpret_cast<mf_f32x4*>(red + (slot * Ly::RQ + 16 * qt + r16) * Ly::RS + 16 * dt + 4 * g) = O[dt][qt];
      if (g == 0) redl[slot * Ly::RQ + 16 * qt + r16] = L[qt][0];
    }
  };
  if constexpr (kWaves > kRedWaves) {
    static_assert(kWaves == 2 * kRedWaves, "two waves per reduction slot");
    if (wave >= kRedWaves) put_partials();
    __syncthreads();
    if (wave < kRedWaves) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        if (qt >= nqt) continue;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const mf_f32x4 o2 =
              *reinterpret_cast<const mf_f32x4*>(red + (slot * Ly::RQ + 16 * qt + r16) * Ly::RS + 16 * dt + 4 * g);
          O[dt][qt] += o2;
        }
        // every lane of a query column holds the same denominator in L[qt][0..3]
        L[qt][0] += redl[slot * Ly::RQ + 16 * qt + r16];
      }
    }
    __syncthreads();
  }
  if (wave < kRedWaves) put_partials();
  __syncthreads();
  constexpr int CPQ = DP / 8;  // 8-column chunks per query
  const float oscale = ldexpf(1.0f, -(t1 + t2));
  for (int idx = tid; idx < nqg * CPQ; idx += kThreads) {
    const int i = idx / CPQ;
    const int c8 = (idx - i * CPQ) * 8;
    if (c8 >= D) continue;
    float l = 0.0f;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < kRedWaves; ++w) {
      l += redl[w * Ly::RQ + i];
      const float4 lo = *reinterpret_cast<const float4*>(red + (w * Ly::RQ + i) * Ly::RS + c8);
      const float4 hi = *reinterpret_cast<const float4*>(red + (w * Ly::RQ + i) * Ly::RS + c8 + 4);
      o[0] += lo.x; o[1] += lo.y; o[2] += lo.z; o[3] += lo.w;
      o[4] += hi.x; o[5] += hi.y; o[6] += hi.z; o[7] += hi.w;
    }
    const bool mass = l > 0.0f;
    const float inv = mass ? oscale / l : 0.0f;
    const int atom = qpre ? q0 + i : int(qidx[q0 + i]);
    const size_t row = size_t(bh) * N + atom;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
    if (p.out) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const T lo = T(o[2 * e]), hi = T(o[2 * e + 1]);
        w[e] = uint32_t(__builtin_bit_cast(uint16_t, lo)) | (uint32_t(__builtin_bit_cast(uint16_t, hi)) << 16);
      }
      const size_t orow = STR ? size_t(b) * p.os_b + size_t(h) * p.os_h + size_t(atom) * p.os_n : row * D;
      *reinterpret_cast<uint4*>(static_cast<T*>(p.out) + orow + c8) = uint4{w[0], w[1], w[2], w[3]};
    }
    if (p.out_f32) {
      float4* dst = reinterpret_cast<float4*>(p.out_f32 + row * D + c8);
      dst[0] = float4{o[0], o[1], o[2], o[3]};
      dst[1] = float4{o[4], o[5], o[6], o[7]};
    }
    if (c8 == 0 && p.lse) p.lse[row] = mass ? ((slow ? s_m[i] : 0.0f) + __log2f(l)) * kLn2 : 0.0f;
  }
  if (claiming) {
    cl->next = claimed_position(p.counter, ticket, reinterpret_cast<const int*>(smem + Ly::kPre)[p.B]);
    cl->claimed = 1;
  }
  __syncthreads();  // the next unit rewrites the index lists and LDS
}

// ---------------------------------------------------------------------------
// schedule: every workgroup derives the same unit list from the masks
// ---------------------------------------------------------------------------
// Nonzero bytes of a dword as bit 7 of each byte: ((x & 0x7f) + 0x7f) | x.
__device__ __forceinline__ uint32_t nz_bytes(uint32_t x) { return (((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x) & 0x80808080u; }

// Bit 7 of each byte in [lo, hi) of a 16-byte chunk (dword j covers bytes 4j..4j+3).
__device__ __forceinline__ uint4 chunk_bytes(int lo, int hi) {
  uint32_t m[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int l = min(max(lo - 4 * j, 0), 4), h = min(max(hi - 4 * j, 0), 4);
    m[j] = h <= l ? 0u : (0x80808080u & (0xffffffffu << (8 * l)) & (0xffffffffu >> (8 * (4 - h))));
  }
  return uint4{m[0], m[1], m[2], m[3]};
}

// Valid (nonzero) byte count of bytes [a, e) of a mask row in global memory,
// and the index of the first zero byte among them (e if none).  The bytes are
// read as the 16-byte aligned chunks that hold them, eight loads in flight; an
// aligned chunk that holds a byte of the row lies on that byte's page.  Every
// chunk is counted whole; the bytes of the first chunk before a are masked
// there (a compile-time slot), and those of the last chunk from e on are read
// again once and taken off.  The first zero is looked for from a on; one past
// e is clamped to e.
__device__ __forceinline__ void scan_row_global(const uint8_t* row, int a, int e, int& count, int& firstzero) {
  firstzero = e;
  if (a >= e) return;
  const uint8_t* begin = row + a;
  const int off = int(reinterpret_cast<uintptr_t>(begin) & 15u);
  const uint8_t* c0 = begin - off;  // pointer arithmetic keeps the global address space
  const int span = off + (e - a);   // bytes from c0 to the end of the segment
  const int nch = (span + 15) >> 4;
  const uint4 keep0 = chunk_bytes(off, 16);
  int cnt = 0, zc = -1;
  uint32_t zw[4] = {0u, 0u, 0u, 0u};
  for (int c = 0; c < nch; c += 8) {
    uint4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t)
      v[t] = c + t < nch ? *reinterpret_cast<const uint4*>(c0 + 16 * (c + t)) : uint4{0u, 0u, 0u, 0u};
    const uint4 m0 = c == 0 ? keep0 : uint4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      uint32_t n0 = nz_bytes(v[t].x), n1 = nz_bytes(v[t].y), n2 = nz_bytes(v[t].z), n3 = nz_bytes(v[t].w);
      uint32_t z0 = n0 ^ 0x80808080u, z1 = n1 ^ 0x80808080u, z2 = n2 ^ 0x80808080u, z3 = n3 ^ 0x80808080u;
      if (t == 0) {
        n0 &= m0.x; n1 &= m0.y; n2 &= m0.z; n3 &= m0.w;
        z0 &= m0.x; z1 &= m0.y; z2 &= m0.z; z3 &= m0.w;
      }
      cnt += __popc(n0) + __popc(n1) + __popc(n2) + __popc(n3);
      if (zc < 0 && (z0 | z1 | z2 | z3) != 0u) {
        zc = c + t;
        zw[0] = z0; zw[1] = z1; zw[2] = z2; zw[3] = z3;
      }
    }
  }
  if (span & 15) {  // bytes e .. of the last chunk
    const uint4 vl = *reinterpret_cast<const uint4*>(c0 + 16 * (nch - 1));
    uint4 ml = chunk_bytes(span & 15, 16);
    if (nch == 1) ml = uint4{ml.x & keep0.x, ml.y & keep0.y, ml.z & keep0.z, ml.w & keep0.w};
    cnt -= __popc(nz_bytes(vl.x) & ml.x) + __popc(nz_bytes(vl.y) & ml.y) + __popc(nz_bytes(vl.z) & ml.z) +
           __popc(nz_bytes(vl.w) & ml.w);
  }
  count += cnt;
  if (zc >= 0) {
    int pos = 12 + (__builtin_ctz(zw[3] | 0x80000000u) >> 3);
    if (zw[2]) pos = 8 + (__builtin_ctz(zw[2]) >> 3);
    if (zw[1]) pos = 4 + (__builtin_ctz(zw[1]) >> 3);
    if (zw[0]) pos = __builtin_ctz(zw[0]) >> 3;
    firstzero = min(e, a - off + 16 * zc + pos);
  }
}

// Valid key / query counts and prefix flags of every molecule into s_info,
// straight from the byte masks in global memory.  Rows are taken in passes of
// whole molecules (row 2m: key mask of molecule m, row 2m + 1: its query
// mask); TPR adjacent threads scan one row, each a segment of it, and the
// segment counts meet over lanes.
template <int DP, bool BIAS>
__device__ __forceinline__ void scan_masks(const Params& p, unsigned char* smem, uint32_t* s_info) {
  constexpr int kThreads = Waves<BIAS>::kCount * 64;
  const int tid = threadIdx.x;
  const int B = p.B, N = p.N;
  const int rows = 2 * B;
  // threads per row: a power of two, <= 8, with rows * tpr <= kThreads when rows allow
  const int tpr = rows > kThreads / 2 ? 1 : rows > kThreads / 4 ? 2 : rows > kThreads / 8 ? 4 : 8;
  const int rpp = kThreads / tpr;  // rows per pass (even)
  int* s_cnt = reinterpret_cast<int*>(smem + Lay<DP, BIAS>::kK2);  // [rpp] counts, then [rpp] first zeros
  static_assert(Lay<DP, BIAS>::kCap * Lay<DP, BIAS>::RB >= kThreads * 2 * 4, "row results must fit in the K2 staging area");
  const int seg = (N + tpr - 1) / tpr;
  for (int r0 = 0; r0 < rows; r0 += rpp) {
    const int r = r0 + tid / tpr, sg = tid & (tpr - 1);
    int cnt = 0, last = N;  // count and first zero byte of the row
    if (r < rows) {
      const uint8_t* row = ((r & 1) ? p.qv : p.pkv) + size_t(r >> 1) * N;
      const int a = min(N, sg * seg);
      scan_row_global(row, a, min(N, a + seg), cnt, last);
    }
    // the tpr threads of a row are adjacent lanes of one wave (all active)
    if (tpr >= 2) {
      cnt = int(AddI32{}(uint32_t(cnt), dpp_peer<0xB1>(uint32_t(cnt))));
      last = int(MinI32{}(uint32_t(last), dpp_peer<0xB1>(uint32_t(last))));
    }
    if (tpr >= 4) {
      cnt = int(AddI32{}(uint32_t(cnt), dpp_peer<0x4E>(uint32_t(cnt))));
      last = int(MinI32{}(uint32_t(last), dpp_peer<0x4E>(uint32_t(last))));
    }
    if (tpr >= 8) {
      cnt = int(AddI32{}(uint32_t(cnt), dpp_peer<0x141>(uint32_t(cnt))));
      last = int(MinI32{}(uint32_t(last), dpp_peer<0x141>(uint32_t(last))));
    }
    if (r < rows && sg == 0) {
      s_cnt[r - r0] = cnt;
      s_cnt[rpp + r - r0] = last;
    }
    __syncthreads();
    const int m0 = r0 >> 1;
    for (int m = tid; m < rpp / 2 && m0 + m < B; m += kThreads) {
      const int ck = min(s_cnt[2 * m], N), cq = min(s_cnt[2 * m + 1], N);
      // the valid bytes are the prefix 0 .. n - 1 exactly when the first zero byte is byte n
      const int zk = s_cnt[rpp + 2 * m], zq = s_cnt[rpp + 2 * m + 1];
      s_info[m0 + m] = uint32_t(ck) | (uint32_t(cq) << 11) | (zk == ck ? kKPre : 0u) | (zq == cq ? kQPre : 0u);
    }
    __syncthreads();
  }
}

// s_order[rank] = molecule, s_pre[rank] = its first list position
// (s_pre[B] = attention units in the list), molecules longest first (cost
// nk^2 x query tiles, ties by index).  A molecule's position is the sum of
// the units of the molecules ranked before it, so rank and position come
// from one pass over (cost, units) pairs: 4 threads per molecule, each over
// every 4th pair.  s_cu holds the pairs (over the staging area).  The
// molecule whose positions hold position w (when w < s_pre[B]) writes
// *s_first = b | (w - its first position) << 16.
template <int W, int GQ, int kCap>
__device__ __forceinline__ void rank_molecules(const Params& p, const uint32_t* s_info, uint16_t* s_order, int* s_pre,
                                               uint2* s_cu, int w, int* s_first) {
  constexpr int kThreads = W * 64;
  const int tid = threadIdx.x;
  const int B = p.B, H = p.H;
  const int B4 = (B + 3) & ~3;
  for (int b = tid; b < B4; b += kThreads) {
    uint2 cu{0u, 0u};  // padding: cost 0 and index >= B never rank before a molecule
    if (b < B) {
      const uint32_t w = s_info[b];
      const int nk = info_nk(w), nq = info_nq(w);
      cu.x = uint32_t(nk * nk) * uint32_t((nq + 15) / 16);
      cu.y = uint32_t(H * num_groups<GQ, kCap>(nk, nq));
    }
    s_cu[b] = cu;
  }
  __syncthreads();
  for (int t = tid; t < 4 * B; t += kThreads) {
    const int b = t >> 2, part = t & 3;
    const uint32_t cb = s_cu[b].x;
    int rank = 0, pre = 0;
    // pairs part, part + 4, ...: two per 16-byte read
    const uint4* c4 = reinterpret_cast<const uint4*>(s_cu);
#pragma unroll 8
    for (int o = 2 * part; o < B4; o += 8) {
      const uint4 v = c4[o >> 1];  // pairs o, o + 1
      const bool f0 = v.x > cb || (v.x == cb && o < b);
      const bool f1 = v.z > cb || (v.z == cb && o + 1 < b);
      rank += int(f0) + int(f1);
      pre += (f0 ? int(v.y) : 0) + (f1 ? int(v.w) : 0);
    }
    // the 4 threads of a molecule are one quad (whole quads are active)
    rank = int(group_reduce<4>(uint32_t(rank), AddI32{}));
    pre = int(group_reduce<4>(uint32_t(pre), AddI32{}));
    if (part == 0) {
      const int units = int(s_cu[b].y);
      s_order[rank] = uint16_t(b);
      s_pre[rank] = pre;
      if (rank == B - 1) s_pre[B] = pre + units;
      if (w >= pre && w < pre + units) *s_first = b | ((w - pre) << 16);
    }
  }
  __syncthreads();
}

// One unit (molecule b, head h, query group g): index lists of non-prefix
// masks and the attention of the group's queries.  Ends with a barrier.
template <typename T, int DP, bool HAS_PV, bool BIAS, bool STR>
__device__ __forceinline__ void run_unit(const Params& p, unsigned char* smem, int b, int h, int g, bool zero_share) {
  using Ly = Lay<DP, BIAS>;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const uint32_t info = reinterpret_cast<const uint32_t*>(smem + Ly::kInfo)[b];
  const int nk = info_nk(info), nq = info_nq(info);
  const bool kpre = (info & kKPre) != 0, qpre = (info & kQPre) != 0;
  const int gs = group_size<Waves<BIAS>::kGroup, Waves<BIAS>::kCap>(nk, nq);
  const int q0 = gs * g;
  const int nqg = min(gs, nq - q0);
  if (nqg > 0) {
    if (!kpre || !qpre) {
      uint16_t* kidx = reinterpret_cast<uint16_t*>(smem + Ly::kKidx);
      uint16_t* qidx = reinterpret_cast<uint16_t*>(smem + Ly::kQidx);
      if (wave == 0 && !kpre) write_ranks(p.pkv + size_t(b) * p.N, p.N, kidx, lane);
      if (wave == 1 && !qpre) write_ranks(p.qv + size_t(b) * p.N, p.N, qidx, lane);
      __syncthreads();
    }
    if (nk > Waves<BIAS>::kCap) unit_body<T, DP, HAS_PV, true, BIAS, STR>(p, smem, b, h, nk, q0, nqg, kpre, qpre, zero_share);
    else unit_body<T, DP, HAS_PV, false, BIAS, STR>(p, smem, b, h, nk, q0, nqg, kpre, qpre, zero_share);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// the kernel: persistent workgroups over the units
// ---------------------------------------------------------------------------
// The list: the attention units (molecule, head, query group) of the
// molecules in cost order (longest first).  Workgroup w takes position w
// first; after that a workgroup that
// finishes a unit claims the next position with one device-scope atomic, so
// the workgroups that finish first take the longest remaining units.
// BIAS: its bias operands take another ~24 KB of LDS (two workgroups per CU still fit).
template <typename T, int DP, bool HAS_PV, bool BIAS, bool STR>
__global__ void __launch_bounds__(Waves<BIAS>::kCount * 64, 2) simplicial_pair_kernel(Params p) {
  constexpr int W = Waves<BIAS>::kCount;
  using Ly = Lay<DP, BIAS>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  uint32_t* s_info = reinterpret_cast<uint32_t*>(smem + Ly::kInfo);
  int* s_pre = reinterpret_cast<int*>(smem + Ly::kPre);
  uint16_t* s_order = reinterpret_cast<uint16_t*>(smem + Ly::kOrder);
  ClaimState* cl = reinterpret_cast<ClaimState*>(smem + Ly::kClaim);
  __shared__ int s_first;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int B = p.B;
  const int G = gridDim.x;
  const int wg = blockIdx.x;

  if (tid == 0) cl->claimed = 0;
  scan_masks<DP, BIAS>(p, smem, s_info);  // ends with a barrier
  rank_molecules<W, Waves<BIAS>::kGroup, Waves<BIAS>::kCap>(p, s_info, s_order, s_pre, reinterpret_cast<uint2*>(smem), wg, &s_first);
  const int total = s_pre[B];

  // the rows of padded queries: a static share of (b, h) pairs per
  // workgroup, written during its first unit (or at once without one)
  if (wg >= total) zero_padded_share<T, DP, STR, Waves<BIAS>::kCount>(p, s_info, wg, G);
  for (int pos = wg; pos < total;) {
    int b, i;  // molecule, unit within it
    if (pos == wg) {
      b = s_first & 0xffff;
      i = s_first >> 16;
    } else {
      // rank of the molecule: the last rank whose prefix is <= pos (the
      // prefixes do not decrease), counted over all ranks at once: lane l
      // compares ranks 4 l .. 4 l + 3 (B <= 256)
      const int4 v = reinterpret_cast<const int4*>(s_pre)[lane];
      const int r0 = 4 * lane;
      const int lo = __popcll(__ballot(r0 < B && v.x <= pos)) + __popcll(__ballot(r0 + 1 < B && v.y <= pos)) +
                     __popcll(__ballot(r0 + 2 < B && v.z <= pos)) + __popcll(__ballot(r0 + 3 < B && v.w <= pos)) - 1;
      b = s_order[lo];
      i = pos - s_pre[lo];
    }
    const uint32_t info = s_info[b];
    const int ng = num_groups<Waves<BIAS>::kGroup, Waves<BIAS>::kCap>(info_nk(info), info_nq(info));
    const int h = div_small(i, ng);
    run_unit<T, DP, HAS_PV, BIAS, STR>(p, smem, b, h, i - h * ng, pos == wg);  // ends with a barrier: cl->next is read
    if (tid == 0) {
      if (cl->claimed) {
        cl->claimed = 0;  // the unit claimed the next position
      } else {
        // every unit run makes exactly one claim (unit_body claims for all
        // units the list holds; this covers a unit without valid queries)
        cl->next = claimed_position(p.counter, atomicAdd(p.counter, 1u), total);
      }
    }
    __syncthreads();
    pos = cl->next;  // rewritten only after the next unit's barriers
  }
}

template <typename T, int DP, bool HAS_PV, bool BIAS, bool STR>
int launch(const Params& prm, int num_cus, hipStream_t stream) {
  const int grid = std::max(8, 2 * num_cus);  // 2 workgroups per CU
  auto kern = simplicial_pair_kernel<T, DP, HAS_PV, BIAS, STR>;
  constexpr int W = Waves<BIAS>::kCount;
  const size_t lds = BIAS ? Lay<DP, BIAS>::kTotalBias : Lay<DP, BIAS>::kTotal;
  static_assert((BIAS ? Lay<DP, BIAS>::kTotalBias : Lay<DP, BIAS>::kTotal) <= 80 * 1024, "two workgroups per CU");
  const int st = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), int(lds));
  if (st != MF_OK) return st;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(W * 64), lds, stream, prm);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

}  // namespace spair

bool simplicial_pair_serves(int tokens, int head_dim, int dtype) {
  return dtype != MF_DTYPE_F32 && head_dim % 8 == 0 && head_dim <= 64 && tokens <= spair::kMaxN;
}

int simplicial_pair_max_batch(int tokens) {
  (void)tokens;
  return spair::kMaxBatch;
}

size_t simplicial_pair_workspace_bytes(int batch, int tokens) {
  (void)batch;
  (void)tokens;
  return spair::kSyncBytes;
}

// One launch over a[0..batch), batch <= simplicial_pair_max_batch(tokens);
// `claims` is the kSyncBytes claim region of the workspace (4-byte aligned,
// 0 before the first launch, left 0 by every launch).
int simplicial_pair_launch(const mf_simplicial_fwd_args* a, void* claims, int num_cus, hipStream_t stream) {
  using namespace spair;
  if (a->batch > simplicial_pair_max_batch(a->tokens))
    return fail(MF_ERR_INVALID_ARGUMENT, "simplicial pair launch: batch slice too large");
  if (!simplicial_pair_serves(a->tokens, a->head_dim, a->dtype))
    return fail(MF_ERR_UNSUPPORTED, "simplicial pair launch: unsupported shape");
  if (a->angle_left != nullptr || a->message_left != nullptr)
    return fail(MF_ERR_UNSUPPORTED, "simplicial pair launch: angle and message terms run on the general kernel");
  Params prm{};
  prm.q = a->q; prm.k1 = a->k1; prm.v1 = a->v1; prm.k2 = a->k2; prm.v2 = a->v2;
  prm.qv = a->query_valid; prm.pkv = a->pair_key_valid; prm.pv = a->pair_valid;
  prm.out = a->out; prm.out_f32 = a->out_f32; prm.lse = a->lse;
  prm.B = a->batch; prm.H = a->heads; prm.N = a->tokens; prm.D = a->head_dim;
  prm.counter = static_cast<unsigned int*>(claims);
  prm.bu = a->bias_u; prm.bv = a->bias_v; prm.bw = a->bias_w; prm.bg = a->bias_gate;
  prm.bias_dtype = a->bias_dtype;
  const long long cb = (long long)a->heads * a->tokens * a->head_dim, ch = (long long)a->tokens * a->head_dim;
  bool fits = true;
  auto strides = [&](const int64_t* st, int& sb, int& sh, int& sn) {
    const bool dflt = st[0] == 0 && st[1] == 0 && st[2] == 0;
    const long long v[3] = {dflt ? cb : st[0], dflt ? ch : st[1], dflt ? a->head_dim : st[2]};
    for (long long x : v) fits = fits && x <= 0x7fffffffLL;
    sb = int(v[0]);
    sh = int(v[1]);
    sn = int(v[2]);
  };
  strides(a->q_stride, prm.qs_b, prm.qs_h, prm.qs_n);
  strides(a->kv_stride, prm.ks_b, prm.ks_h, prm.ks_n);
  strides(a->out_stride, prm.os_b, prm.os_h, prm.os_n);
  if (!fits) return fail(MF_ERR_UNSUPPORTED, "simplicial pair launch: operand strides must be below 2^31 elements");
  const int g = num_cus;
  const bool pv = a->pair_valid != nullptr;
  const bool bf = a->dtype == MF_DTYPE_BF16;
  const bool bias = a->bias_u != nullptr;
  // caller strides: their own instantiations (the contiguous ones keep the shape-derived addressing,
  // which leaves the kernel's scalar registers as they were); none with pair_valid
  bool strided = false;
  for (const int64_t* st : {a->q_stride, a->kv_stride, a->out_stride})
    strided = strided || st[0] != 0 || st[1] != 0 || st[2] != 0;
  if (strided && pv)
    return fail(MF_ERR_UNSUPPORTED, "simplicial pair launch: operand strides are not taken together with pair_valid");
  auto go = [&](auto tag, auto dp, auto has_pv) {
    using T = decltype(tag);
    constexpr int DP = decltype(dp)::value;
    constexpr bool PV = decltype(has_pv)::value;
    if constexpr (!PV) {
      if (strided)
        return bias ? launch<T, DP, false, true, true>(prm, g, stream) : launch<T, DP, false, false, true>(prm, g, stream);
    }
    return bias ? launch<T, DP, PV, true, false>(prm, g, stream) : launch<T, DP, PV, false, false>(prm, g, stream);
  };
  using I32 = std::integral_constant<int, 32>;
  using I64 = std::integral_constant<int, 64>;
  using PV1 = std::true_type;
  using PV0 = std::false_type;
  if (a->head_dim <= 32) {
    if (bf) return pv ? go(__bf16{}, I32{}, PV1{}) : go(__bf16{}, I32{}, PV0{});
    return pv ? go(_Float16{}, I32{}, PV1{}) : go(_Float16{}, I32{}, PV0{});
  }
  if (bf) return pv ? go(__bf16{}, I64{}, PV1{}) : go(__bf16{}, I64{}, PV0{});
  return pv ? go(_Float16{}, I64{}, PV1{}) : go(_Float16{}, I64{}, PV0{});
}

}  // namespace mf

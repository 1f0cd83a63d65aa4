// 2-simplicial attention backward, pair formulation, for bf16 operands and
// head_dim 64 on gfx950 (CDNA4): molecules of at most 80 valid queries and 80
// valid keys, one or two workgroups per (molecule, head), deterministic (no
// floating-point atomics).
//
// The gradient of simplicial_attention.py:206-344 (the quantities of
// triton_simplicial_attention.py:332-782) with the key pairs p = (j, k) as
// the keys of an ordinary attention:
//   W_p = k1_j (.) k2_k,  Z_p = v1_j (.) v2_k,  S_ip = q_i . W_p,
//   P_ip = exp(S_ip - lse_i),  dP_ip = go_i . Z_p,  dS_ip = P_ip (dP_ip - go_i . out_i)
//   dq_i  = sum_p dS_ip W_p                         (contraction over pairs)
//   G_p   = sum_i dS_ip q_i,  H_p = sum_i P_ip go_i   (contractions over queries)
//   dk1_j = sum_k G_jk (.) k2_k,  dk2_k = sum_j G_jk (.) k1_j
//   dv1_j = sum_k H_jk (.) v2_k,  dv2_k = sum_j H_jk (.) v1_j
// Five products of n^3 D multiply-adds, against eleven when every index
// recomputes the scores it owns (simplicial_bwd.hip).
//
// Work split.  The keys are cut into 16-key tiles k0 .. k0 + 15 (outer loop,
// the four waves in step); inside a tile each wave takes the pairs of keys
// (j, j + 1) = (2 jp, 2 jp + 1), jp = wave, wave + 4, ..., and for each pair
// tile (2 j x 16 k = 32 pairs) every 16-query tile:
//   S, dP   C[i][k] = sum_d A[i][d] B[d][k]   A = q / go rows (LDS), B = W / Z
//           of the tile, formed in registers (MFMA 16x16x32 bf16)
//   dq_i   += dS[i][p] W[p][d]   K = the 32 pairs, dS turned through a
//           per-wave LDS scratch (transposed read)
//   G^T, H^T (key x d) += dS^T / P^T [k][i] q / go [i][d]: the S accumulators
//           of two query tiles are the A operand as they are (K = 32 queries)
// then dk1_j / dv1_j (sums over the tile's keys: in-lane over 4 keys, then
// across the four lane groups) go to the wave's own LDS rows of j, and
// dk2 / dv2 of the tile's keys accumulate over the wave's j in registers; at
// the end of the key tile the four waves' partials are added in a fixed
// order.  dq accumulates over every pair in registers and the four waves'
// rows are added in a fixed order at the end.  Every sum has a fixed order:
// two calls give identical bits.
//
// Schedule.  A one-workgroup planning kernel counts every molecule's valid
// keys and queries, marks the molecules this kernel serves (for the
// ownership kernel to skip), and writes the unit list longest first (cost
// ~ j pairs x key tiles x query tiles, the LPT order): molecules with more
// than 40 valid keys run as two units that take alternate key pairs
// (jp = part, part + 2, ...), the others as one.  Workgroup w runs unit w.
// The two halves of a molecule own their dk1 / dv1 rows and hold partial
// sums of dq, dk2 and dv2: part 0 writes its partials to the fp32 gradient
// rows (to its own slab of the workspace when the gradients are bf16), part 1
// to its slab, and a third launch writes part 0 + part 1 in that order.  (Handing the sums over inside the kernel would need
// a device-scope release and acquire per half, which on this part write back
// and invalidate the whole L2 of the XCD and held each workgroup's CU for
// tens of microseconds.)
//
// Precision.  The rows are staged as fp16 scaled by powers of two, one per
// operand and unit, that bring each operand's largest magnitude into [1, 2)
// (bf16 values convert exactly; entries below 2^-14 of the largest lose low
// bits as fp16 subnormals, which moves a dot product by at most 2^-24 of its
// largest term), so that one v_pk_mul_f16 forms two pair products and the
// MFMAs are 16x16x32 f16 with fp32 accumulation:
//   W for S and for dq: k1 k2 rounded to fp16 (the reference backward rounds
//     the score products to bf16, triton_simplicial_attention.py:546-551);
//   Z for dP: hi + lo, both fp16: hi = v1 v2 rounded, lo = fma(v1, v2, -hi),
//     exact (the product of two bf16 values has at most 16 significant
//     bits), since dP - go . out cancels when one pair dominates the softmax
//     (the reference's dP contraction is fp32, :611-645);
//   dS (scaled by 2^-es, es chosen from the operand scales so that
//     |dS| < 2^15 always) and P as MFMA operands: rounded once to fp16;
//   softmax, dS and every accumulator fp32; the scales are undone, exactly,
//   when the gradients are written.
#include <algorithm>
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace pbwd {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int DP = 64;           // head_dim
constexpr int KS = DP + 8;       // bf16 row stride of the staged rows (144 B)
constexpr int kMaxN = 80;        // valid queries and valid keys per molecule
constexpr int NT = kMaxN / 16;   // 16-row tiles
constexpr int SS = 16 + 4;       // bf16 row stride of the dS scratch (40 B)
constexpr int kSlot = 2 * 16 * DP;  // floats of one wave's dk2 / dv2 partial of a key tile

struct Params {
  const __bf16* q;
  const __bf16* k1;
  const __bf16* v1;
  const __bf16* k2;
  const __bf16* v2;
  const __bf16* go;
  const float* out;
  const float* lse;
  const uint8_t* qv;
  const uint8_t* pkv;
  const uint8_t* pv;
  void* dq;               // gradients, fp32 or (gout16) bf16
  void* dk1;
  void* dv1;
  void* dk2;
  void* dv2;
  int gout16;
  const int* total;       // plan: units in the list
  const uint32_t* units;  // plan: (b H + h) << 1 | part, longest first
  const int2* counts;     // plan: [B] valid keys, valid queries
  const uint16_t* lists;  // plan: [B][2][kMaxN] their atoms
  float* slab;            // [B*H][2 parts][5][kMaxN][DP] partial dq, dk2, dv2 of split molecules and (bias)
                          // the dk1, dv1 sums of the unit's keys (compacted rows)
  // factorized bias (BIAS kernels): S += gate_i (u_ij + v_ik + w_jk), u / v / w [B*H, N, N], gate [B*H, N]
  // bf16; gradients fp32 or (gout16) bf16, NULL = not wanted
  const uint16_t* bu;
  const uint16_t* bv;
  const uint16_t* bw;
  const uint16_t* bg;
  void* du;
  void* dvb;
  void* dw;
  void* dgate;
  float* dwpart;          // [B*H][kMaxN j][kMaxN k] dw of the earlier query passes (compacted)
  float* dupart;          // [B*H][kMaxN / 16 key tiles][kMaxN i][kMaxN j] per-key-tile sums over k of dS 2^-es
  float* dvbpart;         // [B*H][2 parts][kMaxN i][kMaxN k] sums over the part's j of dS 2^-es
  float* dgpart;          // [B*H][2 parts][kMaxN i] sums over the part's (j, k) of dS 2^-es (u + v + w)
  float* fds;             // [B*H] 2^es of the unit (dS is carried as dS 2^-es)
  int H, N;
};

// Units per molecule: two halves (alternate key pairs) above 40 valid keys.
__device__ __forceinline__ int parts_of(int nk) { return nk > 40 ? 2 : 1; }

// Relative cost of one unit: j pairs x key tiles x MFMA per (pair tile, all queries).
__device__ __forceinline__ uint32_t unit_cost(int nk, int nq) {
  const int nqt = (nq + 15) / 16;
  return uint32_t((nk + 1) / 2) * uint32_t((nk + 15) / 16) * uint32_t(28 * nqt + 16 * ((nqt + 1) / 2)) /
         uint32_t(parts_of(nk));
}

// Workspace of the pair path (16-byte aligned regions).
struct Ws {
  size_t units, served, counts, lists, slab, dupart, dvbpart, dgpart, fds, dwpart, bytes;
  Ws(int B, int H) {
    const size_t bh = size_t(B) * H;
    units = 16;  // [0, 4): units in the list, [4, 8): molecules the pair kernel does not serve
    served = units + ((bh * 2 * 4 + 15) & ~size_t(15));
    counts = served + ((size_t(B) * 4 + 15) & ~size_t(15));
    lists = counts + size_t(B) * 8;
    slab = (lists + size_t(B) * 2 * kMaxN * 2 + 255) & ~size_t(255);
    dupart = slab + bh * 2 * 5 * kMaxN * DP * 4;
    dvbpart = dupart + bh * (kMaxN / 16) * kMaxN * kMaxN * 4;
    dgpart = dvbpart + bh * 2 * kMaxN * kMaxN * 4;
    fds = dgpart + bh * 2 * kMaxN * 4;
    dwpart = (fds + bh * 4 + 15) & ~size_t(15);
    bytes = dwpart + bh * kMaxN * kMaxN * 4;
  }
};
constexpr int kPlanThreads = 1024;
constexpr int kMaxPlanBatch = 2048;
constexpr int kMaxTokens = 512;  // mask rows the plan reads in one pass of 8 x 64 bytes

struct PlanParams {
  const uint8_t* qv;
  const uint8_t* pkv;
  int* total;       // total[0] units, total[1] unserved molecules
  uint32_t* units;
  int* served;
  int2* counts;     // [B] (valid keys, valid queries)
  uint16_t* lists;  // [B][2][kMaxN] valid key atoms, valid query atoms (when they fit)
  int B, H, N;
};

// LDS layout (bytes).  BIAS: no dk1 / dv1 sums (they run in the workspace) but the bias terms u^T [j][i],
// v^T [k][i] (bf16 as given) and the gates.
constexpr int KU = kMaxN + 8;  // bf16 row stride of u^T, v^T (176 B)
template <bool BIAS>
struct Lay {
  static constexpr size_t rows = 0;                                            // q, go, k1, k2, v1, v2: [80][KS] fp16
  static constexpr size_t acc1 = rows + size_t(6) * kMaxN * KS * 2;            // dk1, dv1 of the wave's j: [2][80][64] f32
  static constexpr size_t slot = acc1 + (BIAS ? 0 : size_t(2) * kMaxN * DP * 4);  // [4 waves][kSlot] f32
  static constexpr size_t dvb = slot + size_t(kWaves) * kSlot * 4;             // BIAS: [4 waves][5][16 k][16 i] f32
  static constexpr size_t scr = dvb + (BIAS ? size_t(kWaves) * NT * 256 * 4 : 0);  // [4 waves][2][32][SS] fp16
  static constexpr size_t ut = scr + size_t(kWaves) * 2 * 32 * SS * 2;         // BIAS: [80][KU] bf16
  static constexpr size_t vt = ut + (BIAS ? size_t(kMaxN) * KU * 2 : 0);      // BIAS: [80][KU] bf16
  static constexpr size_t gt = vt + (BIAS ? size_t(kMaxN) * KU * 2 : 0);      // BIAS: [2][80] f32 gate, gate log2 e
  static constexpr size_t lse2 = gt + (BIAS ? 2 * kMaxN * 4 : 0);              // [80] f32
  static constexpr size_t dlt = lse2 + kMaxN * 4;                              // [80] f32
  static constexpr size_t pvb = dlt + kMaxN * 4;                               // [80][3] u32 pair bits
  static constexpr size_t kidx = pvb + kMaxN * 3 * 4;                          // [80] i32
  static constexpr size_t qidx = kidx + kMaxN * 4;                             // [80] i32
  static constexpr size_t cnt = qidx + kMaxN * 4;                              // [4] i32
  static constexpr size_t red = cnt + 16;                                      // [4 waves][8] u32 operand maxima
  static constexpr size_t con = red + kWaves * 8 * 4;                          // [8] f32 unit constants (kC*)
  static constexpr size_t bytes = con + 8 * 4;
  static_assert(bytes <= 160 * 1024, "one workgroup per CU");
  // BIAS passes of at most 3 query tiles: the four waves' dq partials in slot + dvb
  static_assert(!BIAS || size_t(kWaves) * 48 * DP * 4 <= scr - slot, "dq partials of a pass fit slot + dvb");
  static_assert(size_t(kWaves) * kMaxN * DP * 4 <= scr, "dq partials reuse rows + acc1 / slot");
  static_assert(size_t(kMaxN) * 16 <= size_t(kSlot), "a wave's dv_bias partials of a key tile fit its slot");
  static_assert(48 * 4 <= 2 * 32 * SS * 2, "a wave's dgate partials of a pass fit its scratch");
};

// Unit constants in LDS: S log2 e = S_c cS; dS 2^-es = P (dP_c cP - delta 2^-es); the written gradients are
// the accumulated sums times fDq, fDk1, fDk2, fDv1, fDv2.
enum { kCS = 0, kCP, kFDq, kFDk1, kFDk2, kFDv1, kFDv2, kFDs };

typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 mf_f16x4;

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_u16(uint16_t w) { return __uint_as_float(uint32_t(w) << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 mf_bf16x2;

// One gradient element, fp32 or rounded to bf16.
__device__ __forceinline__ void store_grad(void* base, size_t i, float v, int bf16) {
  if (bf16) static_cast<__bf16*>(base)[i] = __bf16(v);
  else static_cast<float*>(base)[i] = v;
}

// Largest magnitude of eight bf16 (as the 15-bit pattern: for positive values bit order is value order).
__device__ __forceinline__ uint32_t absmax_bits8(const uint4 r) {
  const uint32_t a = max(max(r.x & 0x7fffu, (r.x >> 16) & 0x7fffu), max(r.y & 0x7fffu, (r.y >> 16) & 0x7fffu));
  const uint32_t b = max(max(r.z & 0x7fffu, (r.z >> 16) & 0x7fffu), max(r.w & 0x7fffu, (r.w >> 16) & 0x7fffu));
  return max(a, b);
}

// Exponent of the largest magnitude (its bf16 pattern), 0 for an all-zero operand: scaling by 2^-e puts the
// largest magnitude in [1, 2).
__device__ __forceinline__ int scale_exp(uint32_t bits) { return bits == 0u ? 0 : int((bits >> 7) & 0xffu) - 127; }

// Eight bf16 times 2^-e (exact) as fp16 (exact in the normal fp16 range).
__device__ __forceinline__ uint4 to_f16x8(const uint4 r, float scale) {
  const auto p0 = __builtin_amdgcn_cvt_pkrtz(bf_lo(r.x) * scale, bf_hi(r.x) * scale);
  const auto p1 = __builtin_amdgcn_cvt_pkrtz(bf_lo(r.y) * scale, bf_hi(r.y) * scale);
  const auto p2 = __builtin_amdgcn_cvt_pkrtz(bf_lo(r.z) * scale, bf_hi(r.z) * scale);
  const auto p3 = __builtin_amdgcn_cvt_pkrtz(bf_lo(r.w) * scale, bf_hi(r.w) * scale);
  return uint4{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1), __builtin_bit_cast(uint32_t, p2),
               __builtin_bit_cast(uint32_t, p3)};
}

// Eight fp32 rounded (toward zero) to fp16.
__device__ __forceinline__ mf_f16x8 pack_f16x8(const float* f) {
  const uint4 w{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f[0], f[1])),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f[2], f[3])),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f[4], f[5])),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f[6], f[7]))};
  return __builtin_bit_cast(mf_f16x8, w);
}

__device__ __forceinline__ mf_f16x8 cat8(const mf_f16x4 a, const mf_f16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ mf_f32x4 mma(const mf_f16x8& a, const mf_f16x8& b, const mf_f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads() it does not wait for this thread's
// outstanding global stores (no workgroup reads back what these kernels store to global memory).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// DPP lane moves within rows of 16 (VALU, no LDS): quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Maximum over the wave in every lane: within rows by DPP, across the four rows by the gfx950 lane swaps.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp<kDppXor1>(v));
  v = max(v, dpp<kDppXor2>(v));
  v = max(v, dpp<kDppHalfMirror>(v));
  v = max(v, dpp<kDppMirror>(v));
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = max(uint32_t(a[0]), uint32_t(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return max(uint32_t(b[0]), uint32_t(b[1]));
}

// Sum over each aligned group of 8 lanes, in every lane of the group (pairs, quads, then the two quads).
__device__ __forceinline__ float sum8(float x) {
  x += __uint_as_float(dpp<kDppXor1>(__float_as_uint(x)));
  x += __uint_as_float(dpp<kDppXor2>(__float_as_uint(x)));
  return x + __uint_as_float(dpp<kDppHalfMirror>(__float_as_uint(x)));
}

// Sum over each 16-lane row, in every lane of the row.
__device__ __forceinline__ float row16_sum(float x) {
  x = sum8(x);
  return x + __uint_as_float(dpp<kDppMirror>(__float_as_uint(x)));
}

// Sum over the four 16-lane groups, (g0 + g2) + (g1 + g3) in every lane: the gfx950 lane swaps (VALU, no LDS).
__device__ __forceinline__ float sum_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The unit list (one workgroup).  Mask rows r = 2 b (valid keys of molecule b) and 2 b + 1 (valid queries)
// are read four per wave at a time, every byte load issued before the first ballot; each row's count and, when
// it is at most kMaxN, its list of atoms go to the workspace.  Then the LPT rank of each served molecule (unit
// cost descending, ties by index) and its list positions = prefix sums of the units ranked before it.
__global__ void __launch_bounds__(kPlanThreads) pair_bwd_plan(PlanParams pp) {
  __shared__ uint32_t s_cost[kMaxPlanBatch];
  __shared__ int s_units[kMaxPlanBatch];
  __shared__ int s_count[2 * kMaxPlanBatch];
  __shared__ int s_total, s_unserved;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int B = pp.B, H = pp.H, N = pp.N;
  constexpr int kRows = 4;
  for (int r0 = kRows * wave; r0 < 2 * B; r0 += kRows * (kPlanThreads / 64)) {
    uint8_t v[kRows][kMaxTokens / 64];
    // unconditional loads from clamped addresses (issued back to back), then the out-of-range ones zeroed
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      const int r = min(r0 + rr, 2 * B - 1);
      const uint8_t* row = ((r & 1) ? pp.qv : pp.pkv) + size_t(r >> 1) * N;
#pragma unroll
      for (int sg = 0; sg < kMaxTokens / 64; ++sg) v[rr][sg] = row[min(64 * sg + lane, N - 1)];
    }
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr)
#pragma unroll
      for (int sg = 0; sg < kMaxTokens / 64; ++sg)
        if (64 * sg + lane >= N) v[rr][sg] = uint8_t(0);
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      const int r = r0 + rr;
      if (r >= 2 * B) break;  // uniform
      uint16_t* list = pp.lists + size_t(r >> 1) * 2 * kMaxN + (r & 1) * kMaxN;
      int count = 0;
#pragma unroll
      for (int sg = 0; sg < kMaxTokens / 64; ++sg) {
        const bool on = v[rr][sg] != 0;
        const unsigned long long bal = __ballot(on);
        const int at = count + __popcll(bal & ((1ull << lane) - 1ull));
        if (on && at < kMaxN) list[at] = uint16_t(64 * sg + lane);
        count += __popcll(bal);
      }
      if (lane == 0) s_count[r] = count;
    }
  }
  if (tid == 0) {
    s_total = 0;
    s_unserved = 0;
  }
  lds_barrier();
  for (int b = tid; b < B; b += kPlanThreads) {
    const int nk = s_count[2 * b], nq = s_count[2 * b + 1];
    const bool served = nk > 0 && nq > 0 && nk <= kMaxN && nq <= kMaxN;
    s_cost[b] = served ? unit_cost(nk, nq) : 0u;
    s_units[b] = served ? H * parts_of(nk) : 0;
    pp.served[b] = served ? 1 : 0;
    if (!served && nk > 0 && nq > 0) atomicAdd(&s_unserved, 1);
    pp.counts[b] = int2{nk, nq};
  }
  lds_barrier();
  // rank: kTpm threads per molecule, each over every kTpm-th other molecule, partial sums added over the
  // thread group (adjacent lanes) by shuffles
  const int tpm = B >= kPlanThreads ? 1 : (B > kPlanThreads / 2 ? 2 : (B > kPlanThreads / 4 ? 4 : (B > kPlanThreads / 8 ? 8 : 16)));
  for (int t0 = 0; t0 < B * tpm; t0 += kPlanThreads) {
    const int t = t0 + tid;
    const int b = t / tpm, sub = t % tpm;
    int pre = 0;
    if (b < B) {
      const uint32_t cb = s_cost[b];
      for (int o = sub; o < B; o += tpm)
        if (s_cost[o] > cb || (s_cost[o] == cb && o < b)) pre += s_units[o];
    }
    for (int off = 1; off < tpm; off <<= 1) pre += __shfl_xor(pre, off, 64);
    if (b < B && sub == 0) {
      const int parts = parts_of(s_count[2 * b]);
      for (int u = 0; u < s_units[b]; ++u)
        pp.units[pre + u] = (uint32_t(b * H + u / parts) << 1) | uint32_t(u % parts);
      atomicAdd(&s_total, s_units[b]);
    }
  }
  lds_barrier();
  if (tid == 0) {
    pp.total[0] = s_total;
    pp.total[1] = s_unserved;
  }
}

// The unit's main loop (key tiles x key pairs x NQT query tiles from tile qt0), its dk1 / dv1 rows, dq, and
// for a split molecule the combination of the two halves.  LDS as staged by the kernel.  A unit may run its
// query tiles in passes (first .. last): every key-side sum is linear in the queries, so a later pass adds to
// what the earlier ones left (dk2 / dv2 partials in the unit's slab rows, the dk1 / dv1 sums and dw in the
// workspace, each read back by the thread that wrote it); dq and the query-side bias sums belong to the pass.
template <int NQT, bool BIAS>
__device__ __forceinline__ void unit_body(const Params& p, unsigned char* smem, int nq, int nk, int part, int parts,
                                          int bh, bool has_pv, int qt0, bool first, bool last) {
  using Ly = Lay<BIAS>;
  const int q0 = qt0 * 16;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const size_t rbase = size_t(bh) * p.N;
  // split molecules: part 1's partial dq, dk2, dv2 go to its slab, and part 0's too when the gradients are
  // 16-bit (fp32 ones hold part 0's partials in the gradient rows until the combine launch)
  const bool to_slab = parts == 2 && (part == 1 || p.gout16 != 0);
  float* slab = p.slab + (size_t(bh) * 2 + part) * 5 * kMaxN * DP;
  _Float16* Qs = reinterpret_cast<_Float16*>(smem + Ly::rows);
  _Float16* Gs = Qs + kMaxN * KS;
  _Float16* K1s = Gs + kMaxN * KS;
  _Float16* K2s = K1s + kMaxN * KS;
  _Float16* V1s = K2s + kMaxN * KS;
  _Float16* V2s = V1s + kMaxN * KS;
  float* dk1a = reinterpret_cast<float*>(smem + Ly::acc1);
  float* dv1a = dk1a + kMaxN * DP;
  float* slot = reinterpret_cast<float*>(smem + Ly::slot);
  _Float16* scr = reinterpret_cast<_Float16*>(smem + Ly::scr) + wave * 2 * 32 * SS;
  const float* con = reinterpret_cast<const float*>(smem + Ly::con);
  const float cS = con[kCS], cP = con[kCP];
  const float* lse2 = reinterpret_cast<const float*>(smem + Ly::lse2) + q0;  // the pass's queries
  const float* dlt = reinterpret_cast<const float*>(smem + Ly::dlt) + q0;
  const _Float16* Qp = Qs + q0 * KS;
  const _Float16* Gp = Gs + q0 * KS;
  const uint32_t* pvb = reinterpret_cast<const uint32_t*>(smem + Ly::pvb);
  const int* kidx = reinterpret_cast<const int*>(smem + Ly::kidx);
  const int* qidx = reinterpret_cast<const int*>(smem + Ly::qidx);
  // BIAS: the staged bias terms, and the dk1 / dv1 sums of the unit's keys in the workspace (slab rows 3, 4)
  const uint16_t* uT = reinterpret_cast<const uint16_t*>(smem + Ly::ut) + q0;
  const uint16_t* vT = reinterpret_cast<const uint16_t*>(smem + Ly::vt) + q0;
  const float* cg = reinterpret_cast<const float*>(smem + Ly::gt) + q0;
  float* sk1 = slab + 3 * kMaxN * DP;
  float* sv1 = slab + 4 * kMaxN * DP;
  const int N = p.N;
  // BIAS: the B operand that sums dS over the keys of each j of a pair tile (column c = pair j index)
  const mf_f16x8 jsum = r16 == (g >> 1) ? mf_f16x8{1, 1, 1, 1, 1, 1, 1, 1} : mf_f16x8{0, 0, 0, 0, 0, 0, 0, 0};

  const int nkt = (nk + 15) / 16;
  const int njp = (nk + 1) / 2;
  // BIAS: dgate partial of queries qt 16 + 4 g + r over the lane's (j, k)
  float accg[NQT][4];
#pragma unroll
  for (int t = 0; t < NQT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) accg[t][r] = 0.0f;

  mf_f32x4 dqa[NQT][4];
#pragma unroll
  for (int t = 0; t < NQT; ++t)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) dqa[t][dt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * 16;
    // key k0 + r16 at d = 32 s + 8 g + e: the B operands of S and dP
    mf_f16x8 k2c[2], v2c[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      k2c[s] = *reinterpret_cast<const mf_f16x8*>(K2s + (k0 + r16) * KS + 32 * s + 8 * g);
      v2c[s] = *reinterpret_cast<const mf_f16x8*>(V2s + (k0 + r16) * KS + 32 * s + 8 * g);
    }
    // keys k0 + 8 (g & 1) + e at d = 16 dt + r16: the dq B operand (transposed reads; lane 4 e' + a of a group
    // addresses row e' (+4), columns 4 a .. 4 a + 3)
    mf_f16x8 kcol[4];
    // keys k0 + 4 g + r at d = 16 dt + r16: the dk1 / dv1 sums (BIAS: read in each pair tile's epilogue, which
    // leaves the registers to the bias sums)
    float kk2[4][4], kv2[4][4];
    auto read_kv2 = [&](int dt) {
      const int roff = (k0 + 4 * g + (r16 >> 2)) * KS + 16 * dt + 4 * (r16 & 3);
      const auto a4 = read_tr16(K2s + roff);
      const auto b4 = read_tr16(V2s + roff);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        kk2[dt][r] = float(a4[r]);
        kv2[dt][r] = float(b4[r]);
      }
    };
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const _Float16* pc = K2s + (k0 + 8 * (g & 1) + (r16 >> 2)) * KS + 16 * dt + 4 * (r16 & 3);
      kcol[dt] = cat8(read_tr16(pc), read_tr16(pc + 4 * KS));
      if constexpr (!BIAS) read_kv2(dt);
    }
    // BIAS: this wave's dv_bias partials of the key tile (LDS, [qt][key r16][query 4 g + r])
    float* dvl = reinterpret_cast<float*>(smem + Ly::dvb) + wave * NT * 256;
    if constexpr (BIAS) {
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt)
        *reinterpret_cast<float4*>(dvl + (qt * 16 + r16) * 16 + 4 * g) = float4{0.f, 0.f, 0.f, 0.f};
    }
    mf_f32x4 dk2a[4], dv2a[4];  // key k0 + 4 g + r, d = 16 dt + r16
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      dk2a[dt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
      dv2a[dt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const bool kvalid = k0 + r16 < nk;

    for (int jp = part + parts * wave; jp < njp; jp += parts * kWaves) {
      const int ja = 2 * jp;
      // BIAS: w of pairs (ja + jn, k0 + r16) (clamped indices, unconditional loads), and dw partials
      float wv[2] = {0.0f, 0.0f}, dwa[2] = {0.0f, 0.0f};
      if constexpr (BIAS) {
        const int kc = kidx[min(k0 + r16, nk - 1)];
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) wv[jn] = bf_u16(p.bw[(rbase + kidx[min(ja + jn, nk - 1)]) * N + kc]);
      }
      // the epilogue's LDS operands, read now so that their latency hides under the query loop:
      // k1 / v1 of j = ja + jn at d = 16 dt + r16, and the dk1 / dv1 sums of j so far
      _Float16 k1h[2][4];
      float k1p[2][4], v1p[2][4], d1k[2][4], d1v[2][4];
#pragma unroll
      for (int jn = 0; jn < 2; ++jn)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          k1h[jn][dt] = K1s[(ja + jn) * KS + 16 * dt + r16];
          if constexpr (!BIAS) {
            k1p[jn][dt] = float(k1h[jn][dt]);
            v1p[jn][dt] = float(V1s[(ja + jn) * KS + 16 * dt + r16]);
          }
          if constexpr (BIAS) {
            d1k[jn][dt] = sk1[(ja + jn) * DP + 16 * dt + r16];
            d1v[jn][dt] = sv1[(ja + jn) * DP + 16 * dt + r16];
          } else {
            d1k[jn][dt] = dk1a[(ja + jn) * DP + 16 * dt + r16];
            d1v[jn][dt] = dv1a[(ja + jn) * DP + 16 * dt + r16];
          }
        }
      if constexpr (BIAS) {  // the workspace rows hold sums only after the first key tile (read back by the
                             // g = 0 lanes that wrote them: the same thread, so in order)
        if (kt == 0 && first) {
#pragma unroll
          for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
              d1k[jn][dt] = 0.0f;
              d1v[jn][dt] = 0.0f;
            }
        }
      }
      // ---- the pair tile's operands: W, Z (hi, lo) of pairs (ja + jn, k0 + r16), d = 32 s + 8 g + e ----
      mf_f16x8 wb[2][2], zh[2][2], zl[2][2];
#pragma unroll
      for (int jn = 0; jn < 2; ++jn)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const mf_f16x8 a = *reinterpret_cast<const mf_f16x8*>(K1s + (ja + jn) * KS + 32 * s + 8 * g);
          const mf_f16x8 c = *reinterpret_cast<const mf_f16x8*>(V1s + (ja + jn) * KS + 32 * s + 8 * g);
          wb[jn][s] = a * k2c[s];
          zh[jn][s] = c * v2c[s];
          zl[jn][s] = __builtin_elementwise_fma(c, v2c[s], -zh[jn][s]);
        }
      // W of pairs (ja + (g >> 1), k0 + 8 (g & 1) + e) at d = 16 dt + r16: the dq B operand
      mf_f16x8 wc[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) wc[dt] = kcol[dt] * ((g >> 1) ? k1h[1][dt] : k1h[0][dt]);
      bool pok[2];
#pragma unroll
      for (int jn = 0; jn < 2; ++jn) {
        const int j = ja + jn;
        pok[jn] = kvalid && j < nk && (!has_pv || ((pvb[j * 3 + ((k0 + r16) >> 5)] >> ((k0 + r16) & 31)) & 1u));
      }

      mf_f32x4 gt[2][4], ht[2][4];  // G^T, H^T of the pair tile: key k0 + 4 g + r, d = 16 dt + r16
#pragma unroll
      for (int jn = 0; jn < 2; ++jn)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          gt[jn][dt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
          ht[jn][dt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        }

#pragma unroll
      for (int qb = 0; qb < NQT; qb += 2) {
        // The block's two query tiles side by side (independent chains): S and dP, softmax, dS through the
        // wave's scratch (one slot per tile) for dq.  A tile past NQT carries zeros.
        const int NH = qb + 1 < NQT ? 2 : 1;
        float dsv[2][2][4], pvv[2][2][4];  // [half][jn][r]: query (qb + half) 16 + 4 g + r, key k0 + r16
        mf_f32x4 sacc[2][2], pacc[2][2];
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
          for (int jn = 0; jn < 2; ++jn) {
            sacc[h][jn] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
            pacc[h][jn] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int h = 0; h < NH; ++h) {
            const int qt = qb + h;
            const mf_f16x8 aq = *reinterpret_cast<const mf_f16x8*>(Qp + (qt * 16 + r16) * KS + 32 * s + 8 * g);
            const mf_f16x8 ag = *reinterpret_cast<const mf_f16x8*>(Gp + (qt * 16 + r16) * KS + 32 * s + 8 * g);
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) {
              sacc[h][jn] = mma(aq, wb[jn][s], sacc[h][jn]);
              pacc[h][jn] = mma(ag, zh[jn][s], pacc[h][jn]);
            }
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) pacc[h][jn] = mma(ag, zl[jn][s], pacc[h][jn]);
          }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h >= NH) {
#pragma unroll
            for (int jn = 0; jn < 2; ++jn)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                dsv[h][jn][r] = 0.0f;
                pvv[h][jn][r] = 0.0f;
              }
            continue;
          }
          const int qt = qb + h;
          const float4 l2 = *reinterpret_cast<const float4*>(lse2 + qt * 16 + 4 * g);
          const float4 dl = *reinterpret_cast<const float4*>(dlt + qt * 16 + 4 * g);
          const float l2v[4] = {l2.x, l2.y, l2.z, l2.w};
          const float dlv[4] = {dl.x, dl.y, dl.z, dl.w};
          // BIAS: gate_i (u_ij + v_ik + w_jk) of the lane's queries and pairs (natural units)
          float cl[4] = {0.f, 0.f, 0.f, 0.f}, base[2][4];
          if constexpr (BIAS) {
            // (the offset is opaque to the compiler, so these loads stay here instead of being hoisted out of
            // the loops into registers held throughout)
            int qo = qt * 16 + 4 * g;
            asm volatile("" : "+v"(qo));
            const float4 l4 = *reinterpret_cast<const float4*>(cg + kMaxN + qo);
            cl[0] = l4.x; cl[1] = l4.y; cl[2] = l4.z; cl[3] = l4.w;
            const uint2 v4 = *reinterpret_cast<const uint2*>(vT + (k0 + r16) * KU + qo);
            const float vv[4] = {bf_lo(v4.x), bf_hi(v4.x), bf_lo(v4.y), bf_hi(v4.y)};
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) {
              const uint2 u4 = *reinterpret_cast<const uint2*>(uT + (ja + jn) * KU + qo);
              const float uu[4] = {bf_lo(u4.x), bf_hi(u4.x), bf_lo(u4.y), bf_hi(u4.y)};
#pragma unroll
              for (int r = 0; r < 4; ++r) base[jn][r] = (uu[r] + vv[r]) + wv[jn];
            }
          }
#pragma unroll
          for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float s2 = fmaf(sacc[h][jn][r], cS, -l2v[r]);
              if constexpr (BIAS) s2 = fmaf(cl[r], base[jn][r], s2);
              const float pp = pok[jn] ? fast_exp2(s2) : 0.0f;
              pvv[h][jn][r] = pp;
              dsv[h][jn][r] = pp * fmaf(pacc[h][jn][r], cP, -dlv[r]);
              if constexpr (BIAS) {
                accg[qt][r] = fmaf(dsv[h][jn][r], base[jn][r], accg[qt][r]);
                dwa[jn] = fmaf(cl[r], dsv[h][jn][r], dwa[jn]);
              }
            }
          if constexpr (BIAS) {
            int vo = (qt * 16 + r16) * 16 + 4 * g;
            asm volatile("" : "+v"(vo));
            float4* pv = reinterpret_cast<float4*>(dvl + vo);
            float4 a = *pv;
            a.x += dsv[h][0][0] + dsv[h][1][0];
            a.y += dsv[h][0][1] + dsv[h][1][1];
            a.z += dsv[h][0][2] + dsv[h][1][2];
            a.w += dsv[h][0][3] + dsv[h][1][3];
            *pv = a;
          }
          // dS [pair (jn, key)][query] into slot h of the wave's scratch
#pragma unroll
          for (int jn = 0; jn < 2; ++jn) {
            const uint2 v{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(dsv[h][jn][0], dsv[h][jn][1])),
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(dsv[h][jn][2], dsv[h][jn][3]))};
            *reinterpret_cast<uint2*>(scr + h * 32 * SS + (jn * 16 + r16) * SS + 4 * g) = v;
          }
        }
        __builtin_amdgcn_wave_barrier();
        // dq of queries qt 16 + r16: A = dS [query][pairs (jn = g >> 1, keys 8 (g & 1) + e)] by transposed reads
        mf_f16x8 ads[2];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const _Float16* ps = scr + h * 32 * SS + ((g >> 1) * 16 + 8 * (g & 1) + (r16 >> 2)) * SS + 4 * (r16 & 3);
          ads[h] = cat8(read_tr16(ps), read_tr16(ps + 4 * SS));
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) dqa[qb + h][dt] = mma(ads[h], wc[dt], dqa[qb + h][dt]);
        // BIAS: du partial of (query, j) over the tile's 16 keys: column c < 2 of dS x jsum is the sum for
        // j = ja + c (lanes r16 < 2), written once per key tile
        if constexpr (BIAS) {
          if (p.du != nullptr) {
#pragma unroll
            for (int h = 0; h < NH; ++h) {
              const mf_f32x4 su = mma(ads[h], jsum, mf_f32x4{0.f, 0.f, 0.f, 0.f});
              if (r16 < 2) {
                float* dst = p.dupart + ((size_t(bh) * (kMaxN / 16) + kt) * kMaxN + q0 + (qb + h) * 16 + 4 * g) * kMaxN +
                             ja + r16;
#pragma unroll
                for (int r = 0; r < 4; ++r) dst[r * kMaxN] = su[r];
              }
            }
          }
        }
        // G^T and H^T: A = dS^T / P^T of the two query tiles as the lane holds them (K slot 4 h + r is query
        // (qb + h) 16 + 4 g + r), B = q / go at those queries and d = 16 dt + r16 (transposed reads)
        mf_f16x8 dsb[2], pb[2];
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) {
          float t8[8], u8[8];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            t8[r] = dsv[0][jn][r];
            t8[4 + r] = dsv[1][jn][r];
            u8[r] = pvv[0][jn][r];
            u8[4 + r] = pvv[1][jn][r];
          }
          dsb[jn] = pack_f16x8(t8);
          pb[jn] = pack_f16x8(u8);
        }
        // the second tile's rows when it exists, else the first's again (its K slots carry zeros)
        const int off2 = (qb + 1 < NQT ? 16 : 0) * KS;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const int off = (qb * 16 + 4 * g + (r16 >> 2)) * KS + 16 * dt + 4 * (r16 & 3);
          const mf_f16x8 bq = cat8(read_tr16(Qp + off), read_tr16(Qp + off + off2));
          const mf_f16x8 bg = cat8(read_tr16(Gp + off), read_tr16(Gp + off + off2));
#pragma unroll
          for (int jn = 0; jn < 2; ++jn) {
            gt[jn][dt] = mma(dsb[jn], bq, gt[jn][dt]);
            ht[jn][dt] = mma(pb[jn], bg, ht[jn][dt]);
          }
        }
      }

      // BIAS: dw of the pair tile (sum over the four query groups; each pair belongs to one wave of one unit)
      if constexpr (BIAS) {
        if (p.dw != nullptr) {
          const float fds = con[kFDs] * (1.0f / kLog2e);  // dwa holds sums of gate log2 e dS 2^-es
#pragma unroll
          for (int jn = 0; jn < 2; ++jn) {
            float x = sum_groups(dwa[jn]) * fds;
            if (g == 0 && ja + jn < nk && kvalid) {
              // earlier passes keep their sum in the workspace (read back by the thread that wrote it)
              float* o = p.dwpart + (size_t(bh) * kMaxN + ja + jn) * kMaxN + k0 + r16;
              if (!first) x += *o;
              if (!last) *o = x;
              else store_grad(p.dw, (rbase + kidx[ja + jn]) * N + kidx[k0 + r16], x, p.gout16);
            }
          }
        }
      }
      // ---- the pair tile's key-side gradients ----
      if constexpr (BIAS) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) read_kv2(dt);
#pragma unroll
        for (int jn = 0; jn < 2; ++jn)
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            k1p[jn][dt] = float(k1h[jn][dt]);
            v1p[jn][dt] = float(V1s[(ja + jn) * KS + 16 * dt + r16]);
          }
      }
#pragma unroll
      for (int jn = 0; jn < 2; ++jn) {
        const int j = ja + jn;
        if (j >= nk) continue;  // uniform
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          // dk2 / dv2 of keys k0 + 4 g + r: + k1_j / v1_j (.) G^T / H^T
          // dk1_j / dv1_j at d = 16 dt + r16: sum over the 16 keys (4 in the lane, then the four groups)
          float x = 0.0f, y = 0.0f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            dk2a[dt][r] = fmaf(k1p[jn][dt], gt[jn][dt][r], dk2a[dt][r]);
            dv2a[dt][r] = fmaf(v1p[jn][dt], ht[jn][dt][r], dv2a[dt][r]);
            x = fmaf(kk2[dt][r], gt[jn][dt][r], x);
            y = fmaf(kv2[dt][r], ht[jn][dt][r], y);
          }
          x = sum_groups(x);
          y = sum_groups(y);
          if (g == 0) {  // rows of j belong to this wave
            if constexpr (BIAS) {
              if (kt + 1 < nkt || !last) {
                sk1[j * DP + 16 * dt + r16] = d1k[jn][dt] + x;
                sv1[j * DP + 16 * dt + r16] = d1v[jn][dt] + y;
              } else {  // the last key tile: the gradient rows
                const size_t o = (rbase + kidx[j]) * DP + 16 * dt + r16;
                store_grad(p.dk1, o, (d1k[jn][dt] + x) * con[kFDk1], p.gout16);
                store_grad(p.dv1, o, (d1v[jn][dt] + y) * con[kFDv1], p.gout16);
              }
            } else {
              dk1a[j * DP + 16 * dt + r16] = d1k[jn][dt] + x;
              dv1a[j * DP + 16 * dt + r16] = d1v[jn][dt] + y;
            }
          }
        }
      }
    }

    // ---- dk2 / dv2 of the key tile: the four waves' partials in wave order ----
    {
      float* sl = slot + wave * kSlot;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sl[(4 * g + r) * DP + 16 * dt + r16] = dk2a[dt][r];
          sl[16 * DP + (4 * g + r) * DP + 16 * dt + r16] = dv2a[dt][r];
        }
    }
    lds_barrier();
    for (int u = tid; u < kSlot; u += kThreads) {
      const int which = u / (16 * DP);
      const int kk = (u / DP) % 16;
      const int d = u % DP;
      if (k0 + kk < nk) {
        float s = slot[u] + slot[kSlot + u];
        s += slot[2 * kSlot + u];
        s += slot[3 * kSlot + u];
        s *= which ? con[kFDv2] : con[kFDk2];
        float* ps = slab + size_t(1 + which) * kMaxN * DP + (k0 + kk) * DP + d;
        if (!first) s += *ps;  // an earlier pass's partial (this thread wrote it)
        if (to_slab || !last) *ps = s;
        else store_grad(which ? p.dv2 : p.dk2, (rbase + kidx[k0 + kk]) * DP + d, s, p.gout16);
      }
    }
    // BIAS: dv_bias partial of the key tile (sum over the part's j), the four waves' partials in wave order
    if constexpr (BIAS) {
      if (p.dvb != nullptr) {
        const float* dv0 = reinterpret_cast<const float*>(smem + Ly::dvb);
        for (int u = tid; u < NQT * 256; u += kThreads) {  // key fastest: 64-byte runs of the global rows
          const int kk = u % 16, i16 = (u / 16) % 16, qt = u / 256;
          const int i = q0 + qt * 16 + i16, l = (qt * 16 + kk) * 16 + i16;
          if (i < nq && k0 + kk < nk)
            p.dvbpart[((size_t(bh) * 2 + part) * kMaxN + i) * kMaxN + k0 + kk] =
                ((dv0[l] + dv0[NT * 256 + l]) + dv0[2 * NT * 256 + l]) + dv0[3 * NT * 256 + l];
        }
      }
    }
    lds_barrier();
  }

  if constexpr (BIAS) {
    // dgate partials of the pass: sums over each lane's keys into the wave's own scratch (other waves may still
    // be using theirs), then the four waves in order
    float* gs = reinterpret_cast<float*>(scr);
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = row16_sum(accg[qt][r]);
        if (r16 == 0) gs[qt * 16 + 4 * g + r] = x;
      }
  } else {
    // ---- dk1 / dv1 rows of the unit's keys j (key pairs jp = j / 2 with jp % parts == part) ----
    for (int u = tid; u < nk * DP; u += kThreads) {
      if (((u / DP) >> 1) % parts != part) continue;
      const size_t o = (rbase + kidx[u / DP]) * DP + (u % DP);
      store_grad(p.dk1, o, dk1a[u] * con[kFDk1], p.gout16);
      store_grad(p.dv1, o, dv1a[u] * con[kFDv1], p.gout16);
    }
  }
  lds_barrier();  // rows and acc1 are free for the dq partials
  if constexpr (BIAS) {
    if (p.dgate != nullptr) {
      const float* gs = reinterpret_cast<const float*>(smem + Ly::scr);
      constexpr int kW = 2 * 32 * SS / 2;  // floats per wave's scratch
      for (int i = tid; i < min(nq - q0, NQT * 16); i += kThreads)
        p.dgpart[(size_t(bh) * 2 + part) * kMaxN + q0 + i] =
            ((gs[i] + gs[kW + i]) + gs[2 * kW + i]) + gs[3 * kW + i];
    }
  }
  // ---- dq: the four waves' partials in wave order ----
  // (BIAS: in slot + dvb, since a later pass still needs the rows)
  float* dqs = reinterpret_cast<float*>(smem + (BIAS ? Ly::slot : 0));
  constexpr int kDqs = NQT * 16 * DP;  // one wave's partials
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dqs[wave * kDqs + (qt * 16 + 4 * g + r) * DP + 16 * dt + r16] = dqa[qt][dt][r];
  }
  lds_barrier();
  for (int u = tid; u < min(nq - q0, NQT * 16) * DP; u += kThreads) {
    float s = dqs[u] + dqs[kDqs + u];
    s += dqs[2 * kDqs + u];
    s += dqs[3 * kDqs + u];
    s *= con[kFDq];
    if (to_slab) slab[q0 * DP + u] = s;
    else store_grad(p.dq, (rbase + qidx[q0 + u / DP]) * DP + (u % DP), s, p.gout16);
  }
  if (!last) lds_barrier();  // slot, dvb and the scratch are the next pass's
}

template <bool BIAS>
__global__ void __launch_bounds__(kThreads, 1) pair_bwd_kernel(Params p) {
  using Lk = Lay<BIAS>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  if (int(blockIdx.x) >= *p.total) return;
  const uint32_t unit = p.units[blockIdx.x];
  const int bh = int(unit >> 1);
  const int part = int(unit & 1u);
  const int b = bh / p.H;
  const int N = p.N;
  const int tid = threadIdx.x;
  _Float16* Qs = reinterpret_cast<_Float16*>(smem + Lk::rows);  // q, go, k1, k2, v1, v2 rows in this order
  const int lane = lane_id();
  const int wave = wave_id();
  float* lse2 = reinterpret_cast<float*>(smem + Lk::lse2);
  float* dlt = reinterpret_cast<float*>(smem + Lk::dlt);
  uint32_t* pvb = reinterpret_cast<uint32_t*>(smem + Lk::pvb);
  int* kidx = reinterpret_cast<int*>(smem + Lk::kidx);
  int* qidx = reinterpret_cast<int*>(smem + Lk::qidx);

  // ---- valid keys and queries of molecule b, from the plan (which lists only molecules with 1 .. kMaxN) ----
  const int2 nkq = p.counts[b];
  const int nk = nkq.x, nq = nkq.y;
  if (tid < 2 * kMaxN) {
    const int at = tid < kMaxN ? tid : tid - kMaxN;
    if (at < (tid < kMaxN ? nk : nq)) (tid < kMaxN ? kidx : qidx)[at] = p.lists[size_t(b) * 2 * kMaxN + tid];
  }
  lds_barrier();
  const int parts = parts_of(nk);
  const size_t rbase = size_t(bh) * N;
  // ---- stage q, go, k1, k2, v1, v2 rows (compacted, zero past the counts) as fp16 scaled by 2^-e per operand
  // (e = the exponent of the operand's largest magnitude over the unit), and lse log2 e and
  // delta 2^-es = go . out 2^-es of each query (+inf / 0 on the padding rows: P = 0 there).  Every global
  // load is issued before the first LDS store. ----
  {
    constexpr int kChunks = 6 * kMaxN * 8 / kThreads;  // 16-byte pieces per thread (15)
    constexpr int kDl = (kMaxN * 8 + kThreads - 1) / kThreads;  // (query, 8-d chunk) items per thread (3)
    static_assert(kChunks * kThreads == 6 * kMaxN * 8, "whole passes");
    const __bf16* srcs[6] = {p.q, p.go, p.k1, p.k2, p.v1, p.v2};
    uint4 buf[kChunks];
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int u = tid + kThreads * i;
      const int t = u / (kMaxN * 8);
      const int rr = (u / 8) % kMaxN;
      const int c = u % 8;
      // rows past the count load row 0 (cached) and are zeroed after: no branch around the loads
      const int rrc = rr < (t < 2 ? nq : nk) ? rr : 0;
      const int idx = t < 2 ? qidx[rrc] : kidx[rrc];
      buf[i] = *reinterpret_cast<const uint4*>(srcs[t] + (rbase + idx) * DP + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int u = tid + kThreads * i;
      const int t = u / (kMaxN * 8);
      if ((u / 8) % kMaxN >= (t < 2 ? nq : nk)) buf[i] = uint4{0u, 0u, 0u, 0u};
    }
    uint4 gr[kDl];
    float4 o0[kDl], o1[kDl];
    float lv[kDl];
#pragma unroll
    for (int i = 0; i < kDl; ++i) {
      const int u = tid + kThreads * i;
      const int rr = u / 8, c = u % 8;
      const bool ok = u < kMaxN * 8 && rr < nq;
      const size_t row = rbase + qidx[ok ? rr : 0];
      gr[i] = *reinterpret_cast<const uint4*>(p.go + row * DP + 8 * c);
      o0[i] = *reinterpret_cast<const float4*>(p.out + row * DP + 8 * c);
      o1[i] = *reinterpret_cast<const float4*>(p.out + row * DP + 8 * c + 4);
      lv[i] = p.lse[row] * kLog2e;
      if (!ok) {
        gr[i] = uint4{0u, 0u, 0u, 0u};
        lv[i] = INFINITY;
      }
    }
    // largest magnitude of each operand: per thread, per wave, then over the four waves
    uint32_t mx[6] = {0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int t = (tid + kThreads * i) / (kMaxN * 8);
      const uint32_t m = absmax_bits8(buf[i]);
#pragma unroll
      for (int tt = 0; tt < 6; ++tt) mx[tt] = t == tt ? max(mx[tt], m) : mx[tt];
    }
    uint32_t* red = reinterpret_cast<uint32_t*>(smem + Lk::red);
#pragma unroll
    for (int tt = 0; tt < 6; ++tt) {
      mx[tt] = wave_max_u32(mx[tt]);
      if (lane == 0) red[wave * 8 + tt] = mx[tt];
    }
    lds_barrier();
    int ex[6];
#pragma unroll
    for (int tt = 0; tt < 6; ++tt)
      ex[tt] = scale_exp(max(max(red[tt], red[8 + tt]), max(red[16 + tt], red[24 + tt])));
    // operands q, go, k1, k2, v1, v2 = 0 .. 5; dS is carried as dS 2^-es, |dS| < 2^(eg + ev1 + ev2 + 10)
    const int es = ex[1] + ex[4] + ex[5] - 5;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int u = tid + kThreads * i;
      const int t = u / (kMaxN * 8);
      const int rr = (u / 8) % kMaxN;
      const int c = u % 8;
      int e = ex[0];
#pragma unroll
      for (int tt = 1; tt < 6; ++tt) e = t == tt ? ex[tt] : e;
      *reinterpret_cast<uint4*>(Qs + size_t(t) * kMaxN * KS + rr * KS + 8 * c) = to_f16x8(buf[i], ldexpf(1.0f, -e));
    }
    if (tid == 0) {
      float* con = reinterpret_cast<float*>(smem + Lk::con);
      con[kCS] = ldexpf(kLog2e, ex[0] + ex[2] + ex[3]);
      con[kCP] = ldexpf(1.0f, ex[1] + ex[4] + ex[5] - es);
      con[kFDq] = ldexpf(1.0f, es + ex[2] + ex[3]);
      con[kFDk1] = ldexpf(1.0f, ex[3] + es + ex[0]);
      con[kFDk2] = ldexpf(1.0f, ex[2] + es + ex[0]);
      con[kFDv1] = ldexpf(1.0f, ex[5] + ex[1]);
      con[kFDv2] = ldexpf(1.0f, ex[4] + ex[1]);
      con[kFDs] = ldexpf(1.0f, es);
      if (BIAS && part == 0) p.fds[bh] = con[kFDs];
    }
    const float dscale = ldexpf(1.0f, -es);
#pragma unroll
    for (int i = 0; i < kDl; ++i) {
      const int u = tid + kThreads * i;
      if (kThreads * i >= kMaxN * 8) break;  // whole waves: kMaxN * 8 is a multiple of 64
      const int rr = u / 8, c = u % 8;
      float s = bf_lo(gr[i].x) * o0[i].x;
      s = fmaf(bf_hi(gr[i].x), o0[i].y, s); s = fmaf(bf_lo(gr[i].y), o0[i].z, s);
      s = fmaf(bf_hi(gr[i].y), o0[i].w, s); s = fmaf(bf_lo(gr[i].z), o1[i].x, s);
      s = fmaf(bf_hi(gr[i].z), o1[i].y, s); s = fmaf(bf_lo(gr[i].w), o1[i].z, s);
      s = fmaf(bf_hi(gr[i].w), o1[i].w, s);
      s = sum8(s);
      if (u < kMaxN * 8 && c == 0) {
        dlt[rr] = rr < nq ? s * dscale : 0.0f;
        lse2[rr] = lv[i];
      }
    }
  }
  // ---- pair bits of the compacted keys (pair_valid), 3 words per j ----
  const bool has_pv = p.pv != nullptr;
  if (has_pv) {
    for (int u = tid; u < kMaxN * 3; u += kThreads) {
      const int j = u / 3, w = u % 3;
      uint32_t bits = 0u;
      if (j < nk) {
        const uint8_t* row = p.pv + (size_t(b) * N + kidx[j]) * N;
        for (int t = 0; t < 32; ++t) {
          const int k = 32 * w + t;
          if (k < nk && row[kidx[k]] != 0) bits |= 1u << t;
        }
      }
      pvb[u] = bits;
    }
  }
  if constexpr (BIAS) {
    // ---- u^T [j][i] = u[i][j] and v^T [k][i] = v[i][k] of the compacted atoms (bf16 as given, zero past the
    // counts), the gates and gate log2 e (zero past nq).  Loads from clamped indices, then the selects. ----
    uint16_t* ut = reinterpret_cast<uint16_t*>(smem + Lk::ut);
    uint16_t* vt = reinterpret_cast<uint16_t*>(smem + Lk::vt);
    float* cgs = reinterpret_cast<float*>(smem + Lk::gt);
    constexpr int kPer = 25;  // every load issued before the first LDS store
    static_assert(kMaxN * kMaxN % (kThreads * kPer) == 0, "whole passes");
    for (int u0 = 0; u0 < kMaxN * kMaxN; u0 += kThreads * kPer) {
      uint16_t a[kPer], c[kPer];
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const int u = u0 + tid + kThreads * t;
        const int i = u / kMaxN, j = u % kMaxN;
        const size_t o = (rbase + qidx[min(i, nq - 1)]) * N + kidx[min(j, nk - 1)];
        a[t] = p.bu[o];
        c[t] = p.bv[o];
      }
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const int u = u0 + tid + kThreads * t;
        const int i = u / kMaxN, j = u % kMaxN;
        const bool ok = i < nq && j < nk;
        ut[j * KU + i] = ok ? a[t] : uint16_t(0);
        vt[j * KU + i] = ok ? c[t] : uint16_t(0);
      }
    }
    if (tid < kMaxN) {
      const float gv = bf_u16(p.bg[rbase + qidx[min(tid, nq - 1)]]);
      cgs[tid] = tid < nq ? gv : 0.0f;
      cgs[kMaxN + tid] = tid < nq ? gv * kLog2e : 0.0f;
    }
  } else {
    for (int u = tid; u < 2 * kMaxN * DP / 4; u += kThreads)
      reinterpret_cast<float4*>(smem + Lk::acc1)[u] = float4{0.f, 0.f, 0.f, 0.f};
  }
  lds_barrier();

  if constexpr (BIAS) {  // at most three query tiles per pass (the bias sums leave no registers for more)
    switch ((nq + 15) / 16) {
      case 1: unit_body<1, true>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      case 2: unit_body<2, true>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      case 3: unit_body<3, true>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      case 4:
        unit_body<2, true>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, false);
        unit_body<2, true>(p, smem, nq, nk, part, parts, bh, has_pv, 2, false, true);
        break;
      default:
        unit_body<3, true>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, false);
        unit_body<2, true>(p, smem, nq, nk, part, parts, bh, has_pv, 3, false, true);
        break;
    }
  } else {
    switch ((nq + 15) / 16) {
      case 1: unit_body<1, false>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      case 2: unit_body<2, false>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      case 3: unit_body<3, false>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      case 4: unit_body<4, false>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
      default: unit_body<NT, false>(p, smem, nq, nk, part, parts, bh, has_pv, 0, true, true); break;
    }
  }
}

// Split molecules: part 0's partial dq, dk2, dv2 are in the fp32 gradient rows (or, 16-bit gradients, in its
// slab), part 1's in its slab; write part 0 + part 1 (in that order).  One workgroup per (molecule, head); a
// separate launch, so the stream orders it after both halves without any cross-workgroup fence.
__global__ void __launch_bounds__(kThreads) pair_bwd_combine(Params p) {
  const int bh = blockIdx.x;
  const int b = bh / p.H;
  const int2 nkq = p.counts[b];
  const int nk = nkq.x, nq = nkq.y;
  if (nk <= 0 || nq <= 0 || nk > kMaxN || nq > kMaxN || parts_of(nk) == 1) return;
  const size_t rbase = size_t(bh) * p.N;
  const float* slab0 = p.slab + size_t(bh) * 2 * 5 * kMaxN * DP;
  const float* slab = slab0 + 5 * kMaxN * DP;  // part 1
  const uint16_t* lists = p.lists + size_t(b) * 2 * kMaxN;
  const bool g16 = p.gout16 != 0;
  // rows: dq of the nq queries, then dk2 and dv2 of the nk keys, 16 float4 each; 8 per thread at a time
  const int nrows = nq + 2 * nk;
  for (int u0 = 0; u0 < nrows * 16; u0 += 8 * kThreads) {
    float4 a[8], c[8];
    size_t dst[8];
    void* base[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int u = min(u0 + int(threadIdx.x) + kThreads * i, nrows * 16 - 1);  // clamped: no branch around loads
      const int row = u / 16, q4 = u % 16;
      const int which = row < nq ? 0 : (row < nq + nk ? 1 : 2);
      const int rr = which == 0 ? row : (which == 1 ? row - nq : row - nq - nk);
      const int idx = which == 0 ? lists[kMaxN + rr] : lists[rr];
      base[i] = which == 0 ? p.dq : (which == 1 ? p.dk2 : p.dv2);
      dst[i] = (rbase + idx) * DP + 4 * q4;
      const size_t so = size_t(which) * kMaxN * DP + rr * DP + 4 * q4;
      a[i] = g16 ? *reinterpret_cast<const float4*>(slab0 + so)
                 : *reinterpret_cast<const float4*>(static_cast<const float*>(base[i]) + dst[i]);
      c[i] = *reinterpret_cast<const float4*>(slab + so);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (u0 + int(threadIdx.x) + kThreads * i >= nrows * 16) continue;
      const float4 v{a[i].x + c[i].x, a[i].y + c[i].y, a[i].z + c[i].z, a[i].w + c[i].w};
      if (g16) {
        const uint2 w{__builtin_bit_cast(uint32_t, mf_bf16x2{__bf16(v.x), __bf16(v.y)}),
                      __builtin_bit_cast(uint32_t, mf_bf16x2{__bf16(v.z), __bf16(v.w)})};
        *reinterpret_cast<uint2*>(static_cast<__bf16*>(base[i]) + dst[i]) = w;
      } else {
        *reinterpret_cast<float4*>(static_cast<float*>(base[i]) + dst[i]) = v;
      }
    }
  }
}

// The factorized bias gradients of every served molecule from the units' partial sums (dS 2^-es):
//   du_ij = gate_i 2^es sum_kt dupart[kt][i][j],  dv_ik = gate_i 2^es (part 0 + part 1),
//   dgate_i = 2^es (part 0 + part 1); dw was written by the units.  kFinishSplit workgroups per (molecule,
// head), each thread kFinishBatch entries at a time with every load issued before the first store.
constexpr int kFinishSplit = 4, kFinishBatch = 4;
__global__ void __launch_bounds__(kThreads) pair_bwd_bias_finish(Params p) {
  __shared__ float s_gate[kMaxN];
  __shared__ int s_q[kMaxN], s_k[kMaxN];
  const int bh = blockIdx.x;
  const int b = bh / p.H;
  const int2 nkq = p.counts[b];
  const int nk = nkq.x, nq = nkq.y;
  if (nk <= 0 || nq <= 0 || nk > kMaxN || nq > kMaxN) return;
  const int tid = threadIdx.x;
  const size_t rbase = size_t(bh) * p.N;
  const uint16_t* lists = p.lists + size_t(b) * 2 * kMaxN;
  const float fds = p.fds[bh];
  const bool two = parts_of(nk) == 2;
  if (tid < kMaxN) {
    s_k[tid] = lists[min(tid, nk - 1)];
    s_q[tid] = lists[kMaxN + min(tid, nq - 1)];
    s_gate[tid] = bf_u16(p.bg[rbase + lists[kMaxN + min(tid, nq - 1)]]);
  }
  __syncthreads();
  const float* dvp = p.dvbpart + size_t(bh) * 2 * kMaxN * kMaxN;
  const float* dup = p.dupart + size_t(bh) * (kMaxN / 16) * kMaxN * kMaxN;
  const int n = nq * nk, nkt = (nk + 15) / 16;
  const int step = kThreads * kFinishSplit;
  for (int u0 = blockIdx.y * kThreads + tid; u0 < n; u0 += kFinishBatch * step) {
    float su[kFinishBatch], sv[kFinishBatch];
#pragma unroll
    for (int t = 0; t < kFinishBatch; ++t) {
      const int u = min(u0 + t * step, n - 1);  // clamped: loads without branches
      const int e = (u / nk) * kMaxN + u % nk;
      su[t] = 0.0f;
#pragma unroll
      for (int kt = 0; kt < kMaxN / 16; ++kt) {
        const float x = dup[size_t(kt) * kMaxN * kMaxN + e];
        su[t] += kt < nkt ? x : 0.0f;  // tiles past nkt hold stale workspace bytes
      }
      const float v1 = dvp[kMaxN * kMaxN + e];
      sv[t] = dvp[e] + (two ? v1 : 0.0f);
    }
#pragma unroll
    for (int t = 0; t < kFinishBatch; ++t) {
      const int u = u0 + t * step;
      if (u >= n) break;
      const int i = u / nk, j = u % nk;
      const size_t o = (rbase + s_q[i]) * p.N + s_k[j];
      const float c = s_gate[i] * fds;
      if (p.du != nullptr) store_grad(p.du, o, c * su[t], p.gout16);
      if (p.dvb != nullptr) store_grad(p.dvb, o, c * sv[t], p.gout16);
    }
  }
  if (p.dgate != nullptr && blockIdx.y == 0) {
    const float* gp = p.dgpart + size_t(bh) * 2 * kMaxN;
    for (int i = tid; i < nq; i += kThreads)
      store_grad(p.dgate, rbase + s_q[i], fds * (two ? gp[i] + gp[kMaxN + i] : gp[i]), p.gout16);
  }
}

}  // namespace pbwd

bool simplicial_pair_bwd_serves(const mf_simplicial_bwd_args* a) {
  if (a->dtype != MF_DTYPE_BF16 || a->grad_dtype != MF_DTYPE_BF16 || a->head_dim != pbwd::DP) return false;
  if (a->batch > pbwd::kMaxPlanBatch || a->tokens > pbwd::kMaxTokens || a->workspace == nullptr ||
      reinterpret_cast<uintptr_t>(a->workspace) % 256 != 0 ||
      a->workspace_bytes < pbwd::Ws(a->batch, a->heads).bytes)
    return false;
  if (a->angle_left != nullptr || a->message_left != nullptr) return false;
  if (a->bias_u != nullptr) {  // bf16 bias terms (staged as they are)
    if (a->bias_dtype != MF_DTYPE_BF16 || !a->bias_v || !a->bias_w || !a->bias_gate) return false;
  }
  if (!a->dq || !a->dk1 || !a->dv1 || !a->dk2 || !a->dv2) return false;
  for (const void* ptr : {(const void*)a->q, (const void*)a->k1, (const void*)a->v1, (const void*)a->k2,
                          (const void*)a->v2, (const void*)a->grad_out, (const void*)a->out})
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0) return false;
  return true;
}

int simplicial_pair_bwd_max_tokens() { return pbwd::kMaxN; }

size_t simplicial_pair_bwd_workspace_bytes(int batch, int heads) {
  if (batch <= 0 || heads <= 0 || batch > pbwd::kMaxPlanBatch) return 0;
  return pbwd::Ws(batch, heads).bytes;
}

const int* simplicial_pair_bwd_served(const mf_simplicial_bwd_args* a) {
  const pbwd::Ws ws(a->batch, a->heads);
  return reinterpret_cast<const int*>(static_cast<const unsigned char*>(a->workspace) + ws.served);
}

const int* simplicial_pair_bwd_unserved_count(const mf_simplicial_bwd_args* a) {
  return static_cast<const int*>(a->workspace) + 1;
}

int simplicial_pair_bwd_launch(const mf_simplicial_bwd_args* a, hipStream_t stream) {
  using namespace pbwd;
  if (a->batch > kMaxPlanBatch) return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_bwd: pair plan batch too large");
  const Ws ws(a->batch, a->heads);
  unsigned char* wsp = static_cast<unsigned char*>(a->workspace);
  PlanParams pp{};
  pp.qv = a->query_valid;
  pp.pkv = a->pair_key_valid;
  pp.total = reinterpret_cast<int*>(wsp);
  pp.units = reinterpret_cast<uint32_t*>(wsp + ws.units);
  pp.served = reinterpret_cast<int*>(wsp + ws.served);
  pp.counts = reinterpret_cast<int2*>(wsp + ws.counts);
  pp.lists = reinterpret_cast<uint16_t*>(wsp + ws.lists);
  pp.B = a->batch;
  pp.H = a->heads;
  pp.N = a->tokens;
  Params p{};
  p.total = pp.total;
  p.units = pp.units;
  p.counts = pp.counts;
  p.lists = pp.lists;
  p.slab = reinterpret_cast<float*>(wsp + ws.slab);
  p.q = static_cast<const __bf16*>(a->q);
  p.k1 = static_cast<const __bf16*>(a->k1);
  p.v1 = static_cast<const __bf16*>(a->v1);
  p.k2 = static_cast<const __bf16*>(a->k2);
  p.v2 = static_cast<const __bf16*>(a->v2);
  p.go = static_cast<const __bf16*>(a->grad_out);
  p.out = a->out;
  p.lse = a->lse;
  p.qv = a->query_valid;
  p.pkv = a->pair_key_valid;
  p.pv = a->pair_valid;
  p.dq = a->dq; p.dk1 = a->dk1; p.dv1 = a->dv1; p.dk2 = a->dk2; p.dv2 = a->dv2;
  p.gout16 = a->grads_dtype == MF_DTYPE_BF16 ? 1 : 0;
  const bool bias = a->bias_u != nullptr;
  if (bias) {
    p.bu = static_cast<const uint16_t*>(a->bias_u);
    p.bv = static_cast<const uint16_t*>(a->bias_v);
    p.bw = static_cast<const uint16_t*>(a->bias_w);
    p.bg = static_cast<const uint16_t*>(a->bias_gate);
    p.du = a->du;
    p.dvb = a->dv_bias;
    p.dw = a->dw;
    p.dgate = a->dgate;
    p.dupart = reinterpret_cast<float*>(wsp + ws.dupart);
    p.dvbpart = reinterpret_cast<float*>(wsp + ws.dvbpart);
    p.dgpart = reinterpret_cast<float*>(wsp + ws.dgpart);
    p.fds = reinterpret_cast<float*>(wsp + ws.fds);
    p.dwpart = reinterpret_cast<float*>(wsp + ws.dwpart);
  }
  p.H = a->heads;
  p.N = a->tokens;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  const size_t lds = bias ? Lay<true>::bytes : Lay<false>::bytes;
  const void* kern = bias ? reinterpret_cast<const void*>(pair_bwd_kernel<true>)
                          : reinterpret_cast<const void*>(pair_bwd_kernel<false>);
  if (lds > size_t(dev.max_lds_per_block))
    return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_bwd: the pair kernel needs " + std::to_string(lds) +
                                        " bytes of LDS per workgroup");
  st = ensure_dynamic_lds(kern, int(lds));
  if (st != MF_OK) return st;
  const long long blocks = 2LL * a->batch * a->heads;  // the most units a plan can list
  if (blocks > 0x7fffffffLL) return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_bwd: grid too large");
  hipLaunchKernelGGL(pair_bwd_plan, dim3(1), dim3(kPlanThreads), 0, stream, pp);
  MF_HIP_CHECK(hipGetLastError());
  if (bias) hipLaunchKernelGGL(pair_bwd_kernel<true>, dim3(unsigned(blocks)), dim3(kThreads), lds, stream, p);
  else hipLaunchKernelGGL(pair_bwd_kernel<false>, dim3(unsigned(blocks)), dim3(kThreads), lds, stream, p);
  MF_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(pair_bwd_combine, dim3(unsigned(a->batch * a->heads)), dim3(kThreads), 0, stream, p);
  MF_HIP_CHECK(hipGetLastError());
  if (bias) {
    hipLaunchKernelGGL(pair_bwd_bias_finish, dim3(unsigned(a->batch * a->heads), kFinishSplit), dim3(kThreads), 0,
                       stream, p);
    MF_HIP_CHECK(hipGetLastError());
  }
  return MF_OK;
}

}  // namespace mf

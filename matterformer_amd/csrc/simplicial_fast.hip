// 2-simplicial attention forward for 16-bit operands on gfx950 (CDNA4): the
// kernels behind mf_simplicial_fwd for bf16/fp16 and head_dim <= 64.
//
// Math (simplicial_attention.py:161-180,304-344; triton_simplicial_attention.py:115-329):
//   S_i[j,k] = sum_d q_i[d] k1_j[d] k2_k[d]
//   P_i      = softmax over valid (j,k) of S_i
//   out_i[d] = sum_{j,k} P_i[j,k] v1_j[d] v2_k[d],   lse_i = log sum_{j,k} exp(S_i[j,k])
//
// Two launches on the caller's stream, no host synchronisation:
//   plan   workgroup 0 turns the byte masks into, per molecule, counts of
//          valid keys and queries (and compacted index lists when the valid
//          atoms are not a prefix), and into work items (molecule, head,
//          range of at most 32 valid queries, about work_target logits); the
//          items of molecules with at most CH = 16*NT keys ("small", all of a
//          GEOM-Drugs batch) are listed by estimated time, longest first.
//          The other workgroups of the launch zero the padded query rows.
//   main   a persistent grid (2 workgroups per CU): round r gives small item
//          r G + w to workgroup w for even r and r G + G - 1 - w for odd r,
//          pairing long and short items; then, when tokens > CH, the larger
//          molecules in (j chunk, k chunk) pairs with two sweeps (exact
//          maximum, then accumulation), one query per wave.
// Logical workgroup ids are remapped so that consecutive ids share an XCD
// (blockIdx.x % 8 is the XCD): neighbouring items land in one L2.
//
// Per small item the workgroup stages the keys of (b, h):
//   K1s  [CH][DP+4] fp32 (bf16) / [CH][DP+8] fp16 in LDS (GEMM1 B operand source)
//   V1T  [DP+1][CH+4] fp32 in LDS, transposed, plus a row of key validity
//   Qs   the item's query rows times log2(e), fp32 (bf16) / fp16, in LDS
//   K2 (GEMM1 A operands) and V2 (GEMM2 B operands) in every wave's registers
//        for all of the wave's queries
// Each of the four waves loads a quarter of the 16-key x 32-column tiles of
// K2, V1 and V2 in the MFMA A layout.  V1 and V2 are transposed by an MFMA
// against a 0/1 selector matrix (exact), which leaves each lane with 4
// consecutive keys of one column: one 16-byte LDS store per lane for V1T, and
// the GEMM2 B operand halves for V2.  The K2 and V2 operands go through LDS
// once to reach the other waves.
//
// Per query i and j tile (16 keys j, lane column r16 = j):
//   B1      = bf16(q'_i (.) K1[j])           q' = q log2(e); v_mul_f32 on K1 staged
//                                             as fp32, or v_pk_mul_f16 for fp16
//   GEMM1   C1[k][j] = sum_d K2[k][d] B1[j][d]            (MFMA 16x16x32, k = A rows)
//   P       = exp2(C1)                                     (= exp of the logit)
//   GEMM2   C2[j][d] = sum_k P[j][k] V2[k][d]              (MFMA, P = A operand straight
//                                                          from the C1 registers)
//   out    += sum_j V1[j][d] C2[j][d]         (fp32 FMAs, V1 from LDS)
// The softmax denominator is an extra GEMM2 column whose B operand marks the
// valid keys, so it costs MFMA cycles instead of one VALU add per logit, and
// padded keys need no masking: their K2/V2 rows are zero and their denominator
// entry is 0.  Padded j rows get P = 1 but are weighted by V1 = 0 and
// validity 0.  The code for each count of active 16-key tiles is generated
// separately, so the inner loop is straight-line; the LDS reads of tile j + 1
// are issued before the MFMAs of tile j.
//
// No running maximum in the common case.  With m_d = max_j |K1[j][d]| and
// n_d = max_k |K2[k][d]|, |S_i[j,k]| <= sum_d |q'_i[d]| m_d n_d
// <= |q'_i|_1 max_d (m_d n_d) = U_i.  When U_i <= bound_limit (60 for bf16, 14
// for fp16: P = 2^S then stays a normal number of the operand type and the
// fp32 sums cannot overflow) P = 2^S is used directly: softmax is invariant to
// the offset, and floating point keeps the same relative precision at any
// scale.  Otherwise the query takes two passes: pass 1 computes the exact
// maximum m of the valid logits (GEMM1 only), pass 2 uses P = 2^(S - m) with
// explicit masking (the accumulator starts at -m).
#include <cmath>
#include <type_traits>

#include "mf_common.h"

namespace mf {
namespace sfast {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kPlanThreads = 1024;
constexpr int kMaxBatch = 1024;  // molecules per launch (one plan thread each)
constexpr int kMaxQueriesPerItem = 32;

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_t;
typedef __bf16 bf16x2_e __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_e __attribute__((ext_vector_type(2)));

// Workspace of one launch slice (B molecules of N tokens, H heads), in ints:
//   hdr[4]              n_small_items, n_large_items
//   nkq[B]              molecule info word (see info_*)
//   kidx[B][N]          valid key positions, compacted (only for molecules
//                       whose valid keys are not the prefix 0..nk-1)
//   qidx[B][N]          valid query positions, compacted (likewise)
//   small[MI][4]        items (b, h, q0 | q1 << 16, info) of molecules with nk <= CH
//   large[MI][4]        items of molecules with nk > CH
// with MI = B * H * ceil(N / kWaves), a bound on the item count of either kind.
struct Workspace {
  int* hdr;
  int* nkq;
  int* kidx;
  int* qidx;
  int4* small_items;
  int4* large_items;
};

__host__ __device__ inline size_t max_items(int B, int H, int N) {
  return size_t(B) * H * ((N + kWaves - 1) / kWaves);
}

__host__ __device__ inline Workspace carve_workspace(void* base, int B, int H, int N) {
  Workspace w;
  int* p = static_cast<int*>(base);
  w.hdr = p;
  p += 4;
  w.nkq = p;
  p += B;
  w.kidx = p;
  p += size_t(B) * N;
  w.qidx = p;
  p += size_t(B) * N;
  p += (4 - (reinterpret_cast<uintptr_t>(p) / 4) % 4) % 4;  // 16-byte alignment
  w.small_items = reinterpret_cast<int4*>(p);
  w.large_items = w.small_items + max_items(B, H, N);
  return w;
}

__host__ inline size_t workspace_bytes(int B, int H, int N) {
  return (4 + size_t(B) + 2 * size_t(B) * N + 4) * 4 + 2 * max_items(B, H, N) * sizeof(int4);
}

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
  Workspace ws;
  int B, H, N, D;
  int cap;            // keys per chunk (CH) of the kernel that serves this head dim
  int work_target;    // logits per item
  float bound_limit;  // largest |S| (log2 units) served without a running max
  int vec_ok;         // rows 16-byte aligned and D*2 % 16 == 0
};

// ---------------------------------------------------------------------------
// 16-bit element traits.
// ---------------------------------------------------------------------------
template <typename T>
struct Half;

typedef float f32x2_e __attribute__((ext_vector_type(2)));

template <>
struct Half<__bf16> {
  using Op8 = mf_bf16x8;
  using Op4 = bf16x4_t;
  using Pair = bf16x2_e;
  // K1 is staged in LDS as fp32 so that each product is one v_mul_f32
  using K1T = float;
  struct QOp {
    float q[8];
  };
  __device__ static __forceinline__ mf_f32x4 mfma32(Op8 a, Op8 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_e{lo, hi}, Pair));
  }
  // q is staged as fp32 with log2(e) folded in, so that exp2 of the logits is
  // the softmax numerator and each product q' k1 is rounded to bf16 once
  using QT = float;
  __device__ static __forceinline__ void prepare(Op8 q8, QOp& o) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o.q[e] = float(q8[e]) * kLog2e;
  }
  __device__ static __forceinline__ void store_q(QT* dst, Op8 v) {
    float4* d = reinterpret_cast<float4*>(dst);
    d[0] = float4{float(v[0]) * kLog2e, float(v[1]) * kLog2e, float(v[2]) * kLog2e, float(v[3]) * kLog2e};
    d[1] = float4{float(v[4]) * kLog2e, float(v[5]) * kLog2e, float(v[6]) * kLog2e, float(v[7]) * kLog2e};
  }
  __device__ static __forceinline__ void load_q(const QT* src, QOp& o) {
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    o.q[0] = a.x; o.q[1] = a.y; o.q[2] = a.z; o.q[3] = a.w;
    o.q[4] = b.x; o.q[5] = b.y; o.q[6] = b.z; o.q[7] = b.w;
  }
  __device__ static __forceinline__ float qabs(const QOp& o, int e) { return fabsf(o.q[e]); }
  __device__ static __forceinline__ void store_k1(K1T* dst, Op8 v) {
    float4* d = reinterpret_cast<float4*>(dst);
    d[0] = float4{float(v[0]), float(v[1]), float(v[2]), float(v[3])};
    d[1] = float4{float(v[4]), float(v[5]), float(v[6]), float(v[7])};
  }
  // 8 consecutive d of a K1 row
  struct K1V {
    float4 a, b;
  };
  __device__ static __forceinline__ K1V load_k1(const K1T* k1) {
    return K1V{*reinterpret_cast<const float4*>(k1), *reinterpret_cast<const float4*>(k1 + 4)};
  }
  // bf16(k1 (.) q) for 8 consecutive d: exact fp32 products, rounded once
  __device__ static __forceinline__ Op8 mul_v(const K1V& k, const QOp& o) {
    const uint4 r{pack(k.a.x * o.q[0], k.a.y * o.q[1]), pack(k.a.z * o.q[2], k.a.w * o.q[3]),
                  pack(k.b.x * o.q[4], k.b.y * o.q[5]), pack(k.b.z * o.q[6], k.b.w * o.q[7])};
    return __builtin_bit_cast(Op8, r);
  }
  __device__ static __forceinline__ Op8 mul(const K1T* k1, const QOp& o) { return mul_v(load_k1(k1), o); }
};

template <>
struct Half<_Float16> {
  using Op8 = mf_f16x8;
  using Op4 = f16x4_t;
  using Pair = f16x2_e;
  using K1T = _Float16;
  struct QOp {
    f16x2_e pair[4];
  };
  __device__ static __forceinline__ mf_f32x4 mfma32(Op8 a, Op8 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_e{lo, hi}, Pair));
  }
  // q is staged as fp16(q log2 e)
  using QT = _Float16;
  __device__ static __forceinline__ void prepare(Op8 q8, QOp& o) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
      o.pair[p] = f16x2_e{_Float16(float(q8[2 * p]) * kLog2e), _Float16(float(q8[2 * p + 1]) * kLog2e)};
  }
  __device__ static __forceinline__ void store_q(QT* dst, Op8 v) {
    Op8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = _Float16(float(v[e]) * kLog2e);
    *reinterpret_cast<Op8*>(dst) = r;
  }
  __device__ static __forceinline__ void load_q(const QT* src, QOp& o) {
    const uint4 w = *reinterpret_cast<const uint4*>(src);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) o.pair[p] = __builtin_bit_cast(f16x2_e, ws[p]);
  }
  __device__ static __forceinline__ float qabs(const QOp& o, int e) {
    return fabsf(float((e & 1) ? o.pair[e >> 1].y : o.pair[e >> 1].x));
  }
  __device__ static __forceinline__ void store_k1(K1T* dst, Op8 v) { *reinterpret_cast<Op8*>(dst) = v; }
  struct K1V {
    uint4 w;
  };
  __device__ static __forceinline__ K1V load_k1(const K1T* k1) { return K1V{*reinterpret_cast<const uint4*>(k1)}; }
  // fp16(k1 (.) q) with v_pk_mul_f16 (correctly rounded products)
  __device__ static __forceinline__ Op8 mul_v(const K1V& k, const QOp& o) {
    const uint32_t ws[4] = {k.w.x, k.w.y, k.w.z, k.w.w};
    uint32_t r[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) r[p] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_e, ws[p]) * o.pair[p]);
    return __builtin_bit_cast(Op8, uint4{r[0], r[1], r[2], r[3]});
  }
  __device__ static __forceinline__ Op8 mul(const K1T* k1, const QOp& o) { return mul_v(load_k1(k1), o); }
};


__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// LDS geometry of the main kernels (host sizing and device carving).
template <typename T, int DP, int NT>
struct Layout {
  using K1T = typename Half<T>::K1T;
  static constexpr int CH = 16 * NT;         // keys per chunk
  using QT = typename Half<T>::QT;
  static constexpr int KS = DP + 16 / int(sizeof(QT));  // row stride (elements) of Qs
  static constexpr int K1S = DP + 16 / int(sizeof(K1T));  // row stride (elements) of K1s
  static constexpr int VS = CH + 8;          // row stride (elements) of V2T
  static constexpr int WS = CH + 4;          // row stride (floats) of V1T
  static constexpr int PW = (CH + 31) / 32;  // pair-valid words per row
  static constexpr size_t kK1 = 0;
  static constexpr size_t kV2T = kK1 + size_t(CH) * K1S * sizeof(K1T);
  // the small items keep the GEMM2 B operands (DP/16 x NPR operands of 16
  // bytes per lane) where the larger molecules keep V2T
  static constexpr size_t kVBBytes = size_t(DP / 16) * ((NT + 1) / 2) * 64 * 16;
  static constexpr size_t kV2TBytes = size_t(DP) * VS * sizeof(T);
  static constexpr size_t kV1T = (kV2T + (kVBBytes > kV2TBytes ? kVBBytes : kV2TBytes) + 15) & ~size_t(15);
  static constexpr size_t kQs = kV1T + size_t(DP + 1) * WS * 4;  // V1T rows: DP columns + key validity
  static constexpr size_t kPV = kQs + size_t(kMaxQueriesPerItem) * KS * sizeof(QT);
  static constexpr size_t kAB = kPV + size_t(CH) * PW * 4;
  static constexpr size_t kRed2 = kAB + size_t(DP) * 4;              // per-wave column maxima of |K2|
  static constexpr size_t kRed = kRed2 + size_t(kWaves) * DP * 4;    // per-wave column maxima of |K1|
  static constexpr size_t kQn = kRed + size_t(kWaves) * DP * 4;      // |q'|_1 of the item's queries
  static constexpr size_t kKA = (kQn + size_t(kMaxQueriesPerItem) * 4 + 15) & ~size_t(15);
  // small items: the K2 GEMM1 A operands (NT x DP/32 operands of 16 bytes per lane)
  static constexpr size_t kFixed = kKA + size_t(NT) * (DP / 32) * 64 * 16;
};

// max over the valid logits of one 16-row j tile (log2 units, -inf if none);
// NKT = number of 16-key tiles of the current key chunk.
template <typename T, int DP, int NT, int NKT, bool HAS_PV>
__device__ __forceinline__ float jtile_max(const typename Half<T>::K1T* K1s, const uint32_t* pvb,
                                           const typename Half<T>::Op8 (&ka)[NT][DP / 32],
                                           const typename Half<T>::QOp (&qo)[DP / 32], int jt, int nkj, int nkk,
                                           int g, int r16) {
  using Hf = Half<T>;
  using Op8 = typename Hf::Op8;
  using L = Layout<T, DP, NT>;
  constexpr int NCH = DP / 32;
  const int j = jt * 16 + r16;
  Op8 b1[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) b1[c] = Hf::mul(K1s + j * L::K1S + c * 32 + g * 8, qo[c]);
  uint32_t pw[L::PW];
  if constexpr (HAS_PV) {
#pragma unroll
    for (int w = 0; w < L::PW; ++w) pw[w] = pvb[j * L::PW + w];
  }
  float mloc = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) {
    mf_f32x4 sv = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) sv = Hf::mfma32(ka[kt][c], b1[c], sv);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = kt * 16 + 4 * g + r;
      bool ok = j < nkj && k < nkk;
      if constexpr (HAS_PV) ok = ok && ((pw[kt >> 1] >> ((kt & 1) * 16 + 4 * g + r)) & 1u);
      if (ok) mloc = fmaxf(mloc, sv[r]);
    }
  }
  return mloc;
}

// acc[nt] += sum over this j tile of V1 (.) (P V2), with P = 2^(S - m).
// MASKED: explicit masking of padded j/k (required whenever m != 0).  Without
// it, padded keys get P = 1 (their K2 rows are zero) but meet zero V2 rows and
// a zero in `ones_edge`, the denominator operand of the last key pair.
template <typename T, int DP, int NT, int NKT, bool HAS_PV, bool MASKED>
__device__ __forceinline__ void jtile_acc(const typename Half<T>::K1T* K1s, const float* V1T, const uint32_t* pvb,
                                          const typename Half<T>::Op8 (&ka)[NT][DP / 32],
                                          const typename Half<T>::Op8 (&vb)[DP / 16][(NT + 1) / 2],
                                          typename Half<T>::Op8 ones_full, typename Half<T>::Op8 ones_edge,
                                          const typename Half<T>::QOp (&qo)[DP / 32], int jt, int nkj, int nkk,
                                          float m, float (&acc)[DP / 16 + 1], int g, int r16) {
  using Hf = Half<T>;
  using Op8 = typename Hf::Op8;
  using L = Layout<T, DP, NT>;
  constexpr int NCH = DP / 32;
  constexpr int ND = DP / 16;
  constexpr int NPU = (NKT + 1) / 2;  // 32-key GEMM2 steps in use
  const int j = jt * 16 + r16;
  Op8 b1[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) b1[c] = Hf::mul(K1s + j * L::K1S + c * 32 + g * 8, qo[c]);
  uint32_t pw[L::PW];
  if constexpr (HAS_PV) {
#pragma unroll
    for (int w = 0; w < L::PW; ++w) pw[w] = pvb[j * L::PW + w];
  }
  // GEMM1 and P = 2^(S - m), packed straight into the GEMM2 A operands
  uint32_t pa[NPU][4];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) {
    mf_f32x4 sv = mf_f32x4{-m, -m, -m, -m};
#pragma unroll
    for (int c = 0; c < NCH; ++c) sv = Hf::mfma32(ka[kt][c], b1[c], sv);
    float pe[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float e = fast_exp2(sv[r]);
      if constexpr (MASKED) {
        const int k = kt * 16 + 4 * g + r;
        e = (j < nkj && k < nkk) ? e : 0.0f;
      }
      if constexpr (HAS_PV) e = ((pw[kt >> 1] >> ((kt & 1) * 16 + 4 * g + r)) & 1u) ? e : 0.0f;
      pe[r] = e;
    }
    pa[kt >> 1][(kt & 1) * 2 + 0] = Hf::pack(pe[0], pe[1]);
    pa[kt >> 1][(kt & 1) * 2 + 1] = Hf::pack(pe[2], pe[3]);
  }
  if constexpr (NKT % 2 == 1) {
    pa[NPU - 1][2] = 0u;
    pa[NPU - 1][3] = 0u;
  }
  // GEMM2 (C2[j][d] = sum_k P[j][k] V2[k][d]) and the V1 epilogue
#pragma unroll
  for (int nt = 0; nt <= ND; ++nt) {
    mf_f32x4 c2 = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pr = 0; pr < NPU; ++pr) {
      const Op8 a = __builtin_bit_cast(Op8, uint4{pa[pr][0], pa[pr][1], pa[pr][2], pa[pr][3]});
      const Op8 bop = nt < ND ? vb[nt < ND ? nt : 0][pr] : (pr == NPU - 1 ? ones_edge : ones_full);
      c2 = Hf::mfma32(a, bop, c2);
    }
    const float4 v1 = *reinterpret_cast<const float4*>(V1T + (nt < ND ? nt * 16 + r16 : DP) * L::WS + jt * 16 + 4 * g);
    acc[nt] += v1.x * c2[0] + v1.y * c2[1] + v1.z * c2[2] + v1.w * c2[3];
  }
}

// acc += the contributions of j tiles 0 .. NKT-1 of one query (all of a small
// item's keys): jtile_acc with the LDS reads software-pipelined.  The K1 rows
// of tile jt + 1 are read while tile jt runs its GEMMs, and the V1 columns of
// tile jt are read at its start, so that no LDS read waits in the middle of
// the MFMA chain.
template <typename T, int DP, int NT, int NKT, bool HAS_PV, bool MASKED>
__device__ __forceinline__ void query_acc(const typename Half<T>::K1T* K1s, const float* V1T, const uint32_t* pvb,
                                          const typename Half<T>::Op8 (&ka)[NT][DP / 32],
                                          const typename Half<T>::Op8 (&vb)[DP / 16][(NT + 1) / 2],
                                          typename Half<T>::Op8 ones_full, typename Half<T>::Op8 ones_edge,
                                          const typename Half<T>::QOp (&qo)[DP / 32], int nk, float m,
                                          float (&acc)[DP / 16 + 1], int g, int r16) {
  using Hf = Half<T>;
  using Op8 = typename Hf::Op8;
  using L = Layout<T, DP, NT>;
  constexpr int NCH = DP / 32;
  constexpr int ND = DP / 16;
  constexpr int NPU = (NKT + 1) / 2;
  typename Hf::K1V k1[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) k1[c] = Hf::load_k1(K1s + r16 * L::K1S + c * 32 + g * 8);
#pragma unroll 1
  for (int jt = 0; jt < NKT; ++jt) {
    const int j = jt * 16 + r16;
    float4 v1[ND + 1];
#pragma unroll
    for (int nt = 0; nt <= ND; ++nt)
      v1[nt] = *reinterpret_cast<const float4*>(V1T + (nt < ND ? nt * 16 + r16 : DP) * L::WS + jt * 16 + 4 * g);
    Op8 b1[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) b1[c] = Hf::mul_v(k1[c], qo[c]);
    // next tile's K1 rows (the last tile re-reads its own rows)
    const int jn = jt + 1 < NKT ? j + 16 : j;
#pragma unroll
    for (int c = 0; c < NCH; ++c) k1[c] = Hf::load_k1(K1s + jn * L::K1S + c * 32 + g * 8);
    // keep the reads above ahead of the MFMA chain (the scheduler would sink
    // them next to their uses)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t pw[L::PW];
    if constexpr (HAS_PV) {
#pragma unroll
      for (int w = 0; w < L::PW; ++w) pw[w] = pvb[j * L::PW + w];
    }
    uint32_t pa[NPU][4];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      mf_f32x4 sv = mf_f32x4{-m, -m, -m, -m};
#pragma unroll
      for (int c = 0; c < NCH; ++c) sv = Hf::mfma32(ka[kt][c], b1[c], sv);
      float pe[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float e = fast_exp2(sv[r]);
        if constexpr (MASKED) {
          const int k = kt * 16 + 4 * g + r;
          e = (j < nk && k < nk) ? e : 0.0f;
        }
        if constexpr (HAS_PV) e = ((pw[kt >> 1] >> ((kt & 1) * 16 + 4 * g + r)) & 1u) ? e : 0.0f;
        pe[r] = e;
      }
      pa[kt >> 1][(kt & 1) * 2 + 0] = Hf::pack(pe[0], pe[1]);
      pa[kt >> 1][(kt & 1) * 2 + 1] = Hf::pack(pe[2], pe[3]);
    }
    if constexpr (NKT % 2 == 1) {
      pa[NPU - 1][2] = 0u;
      pa[NPU - 1][3] = 0u;
    }
    mf_f32x4 c2[ND + 1];
#pragma unroll
    for (int nt = 0; nt <= ND; ++nt) {
      c2[nt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pr = 0; pr < NPU; ++pr) {
        const Op8 a = __builtin_bit_cast(Op8, uint4{pa[pr][0], pa[pr][1], pa[pr][2], pa[pr][3]});
        const Op8 bop = nt < ND ? vb[nt < ND ? nt : 0][pr] : (pr == NPU - 1 ? ones_edge : ones_full);
        c2[nt] = Hf::mfma32(a, bop, c2[nt]);
      }
    }
#pragma unroll
    for (int nt = 0; nt <= ND; ++nt) {
      acc[nt] = fmaf(v1[nt].x, c2[nt][0], acc[nt]);
      acc[nt] = fmaf(v1[nt].y, c2[nt][1], acc[nt]);
      acc[nt] = fmaf(v1[nt].z, c2[nt][2], acc[nt]);
      acc[nt] = fmaf(v1[nt].w, c2[nt][3], acc[nt]);
    }
  }
}

// Maximum over the lanes l ^ OFF, l ^ OFF/2, ... (log2 NV steps) of NV
// values per lane, scattered: each step keeps half of the values, so the
// lane ends with the maximum of value idx (NV - 1 shuffles instead of
// NV log2 NV).
template <int NV, int OFF>
__device__ __forceinline__ float reduce_scatter_max(const float (&v)[NV], int lane, int& idx) {
  if constexpr (NV == 1) {
    idx = 0;
    return v[0];
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
    const float r = reduce_scatter_max<NV / 2, OFF / 2>(k, lane, sub);
    idx = (up ? NV / 2 : 0) + sub;
    return r;
  }
}

// Calls f(std::integral_constant<int, n>) for the runtime n in [1, NT].
template <int NT, int I = 1, typename F>
__device__ __forceinline__ void with_tiles(int n, F&& f) {
  if constexpr (I <= NT) {
    if (n == I) {
      f(std::integral_constant<int, I>{});
    } else {
      with_tiles<NT, I + 1>(n, static_cast<F&&>(f));
    }
  }
}

// ---------------------------------------------------------------------------
// plan: one workgroup of kPlanThreads builds the workspace.
// ---------------------------------------------------------------------------
// Molecule info word: nk | kpre << 30 | qpre << 31 in item.w, and
// nq | nk << 15 | kpre << 30 | qpre << 31 in nkq[b]; kpre / qpre: the valid
// keys / queries are exactly the prefix 0..n-1 (no index list needed).
__device__ __forceinline__ int info_nq(uint32_t w) { return int(w & 0x7fffu); }
__device__ __forceinline__ int info_nk(uint32_t w) { return int((w >> 15) & 0x7fffu); }
constexpr uint32_t kKPre = 1u << 30;
constexpr uint32_t kQPre = 1u << 31;

__device__ __forceinline__ int plan_queries_per_item(int nk, int cls, int work_target) {
  if (cls) return kWaves;
  int qpi = max(kWaves, min(work_target / max(nk * nk, 1), kMaxQueriesPerItem));
  return qpi - qpi % kWaves;
}

// The aligned dword at window offset base + 4 lane of a mask row (0 past the
// row).  A dword that starts inside [row - off, row + N) stays on the row's
// pages.
__device__ __forceinline__ uint32_t load_window(const uint8_t* row, int N, int base, int lane, int& off) {
  const uintptr_t start = reinterpret_cast<uintptr_t>(row);
  const uintptr_t astart = start & ~uintptr_t(3);
  off = int(start - astart);
  const int boff = base + 4 * lane;
  return boff < off + N ? *reinterpret_cast<const uint32_t*>(astart + boff) : 0u;
}

// Valid bytes of one window (the dword w of each lane, bytes of lane l at
// atoms t = boff + e - off) added to `count`, and the last valid atom so far
// in `last`.  The valid atoms are a prefix exactly when last + 1 == count.
__device__ __forceinline__ void scan_window(uint32_t w, int boff, int off, int N, int& count, int& last) {
  int ll = -1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = boff + e - off;
    const bool v = t >= 0 && t < N && ((w >> (8 * e)) & 0xffu) != 0u;
    count += __popcll(__ballot(v));
    ll = v ? t : ll;
  }
  const unsigned long long any = __ballot(ll >= 0);
  if (any) last = __builtin_amdgcn_readlane(ll, 63 - __builtin_clzll(any));
}

// dst[r] = the atom of valid rank r in a mask row (one wave).
__device__ void write_ranks(const uint8_t* row, int N, int* dst, int lane) {
  const unsigned long long below = (1ull << lane) - 1ull;
  int run = 0;
#pragma unroll 1
  for (int t0 = 0; t0 < N; t0 += 64) {
    const int t = t0 + lane;
    const bool ok = t < N && row[t] != 0;
    const unsigned long long bal = __ballot(ok);
    if (ok) dst[run + __popcll(bal & below)] = t;
    run += __popcll(bal);
  }
}

// Rows of padded queries are zeroed by workgroups 1.. of the plan launch,
// concurrently with the plan itself (workgroup 0): one 16-byte chunk of the
// 16-bit output per thread and step, rows (b, h, i) in b-major order.
__device__ void zero_padded_rows(const Params& p, int worker, int workers) {
  const int per_row = p.D / 8;  // head_dim % 8 == 0 on this path
  const int rows_per_step = kPlanThreads / per_row;
  const long long rows = (long long)p.B * p.H * p.N;
  const int rr = threadIdx.x / per_row, c = threadIdx.x - rr * per_row;
  if (rr >= rows_per_step) return;
#pragma unroll 1
  for (long long row = (long long)worker * rows_per_step + rr; row < rows; row += (long long)workers * rows_per_step) {
    const long long bh = row / p.N;
    const int i = int(row - bh * p.N);
    if (p.qv[(bh / p.H) * p.N + i]) continue;
    if (p.vec_ok) {
      if (p.out) reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + row * p.D)[c] = uint4{0u, 0u, 0u, 0u};
      if (p.out_f32) {
        float4* o = reinterpret_cast<float4*>(p.out_f32 + row * p.D);
        o[2 * c] = float4{0.f, 0.f, 0.f, 0.f};
        o[2 * c + 1] = float4{0.f, 0.f, 0.f, 0.f};
      }
    } else {
      // outputs not 16-byte aligned (operands are, on this path): element stores
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (p.out) static_cast<uint16_t*>(p.out)[row * p.D + 8 * c + e] = 0;
        if (p.out_f32) p.out_f32[row * p.D + 8 * c + e] = 0.0f;
      }
    }
    if (c == 0 && p.lse) p.lse[row] = 0.0f;
  }
}

// Items of one molecule: queries per item, item count and, for small
// molecules, the cost keys of its full items and of its last item (the query
// loop's steps per wave, ceil(queries / kWaves) x key tiles).
constexpr int kCostKeys = 64;
struct MolItems {
  int cls, qpi, splits, n, key_full, key_last;
};
__device__ __forceinline__ MolItems mol_items(uint32_t w, int H, int cap, int work_target) {
  MolItems m;
  const int nk = info_nk(w), nq = info_nq(w);
  m.cls = nk > cap ? 1 : 0;
  m.qpi = plan_queries_per_item(nk, m.cls, work_target);
  m.splits = (nq + m.qpi - 1) / m.qpi;
  m.n = H * m.splits;
  const int nkt = (nk + 15) / 16;
  const int q_last = nq - (m.splits - 1) * m.qpi;
  m.key_full = min(kCostKeys - 1, ((m.qpi + kWaves - 1) / kWaves) * nkt);
  m.key_last = min(kCostKeys - 1, ((q_last + kWaves - 1) / kWaves) * nkt);
  return m;
}

__global__ void __launch_bounds__(kPlanThreads) simplicial_plan_kernel(Params p) {
  if (blockIdx.x > 0) {
    zero_padded_rows(p, blockIdx.x - 1, gridDim.x - 1);
    return;
  }
  constexpr int kPlanWaves = kPlanThreads / 64;
  __shared__ uint32_t s_info[kMaxBatch];
  __shared__ int s_cnt[kCostKeys];  // small items per cost key, then the next position of each key
  __shared__ int s_small, s_large, s_large_next;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int B = p.B, H = p.H, N = p.N;
  const Workspace& ws = p.ws;
  if (tid < kCostKeys) s_cnt[tid] = 0;
  if (tid == 0) s_small = s_large = s_large_next = 0;

  // 1. valid keys / queries per molecule and whether they form a prefix (one
  //    wave per molecule).  Rows of up to 252 bytes are one window: the
  //    windows of kRound molecules are loaded before any is scanned.
  constexpr int kRound = 4;
  auto put_info = [&](int b, int ck, int lk, int cq, int lq) {
    if (lane == 0)
      s_info[b] = uint32_t(cq) | (uint32_t(ck) << 15) | (lk + 1 == ck ? kKPre : 0u) | (lq + 1 == cq ? kQPre : 0u);
  };
  if (N <= 252) {
#pragma unroll 1
    for (int b0 = wave; b0 < B; b0 += kPlanWaves * kRound) {
      uint32_t wk[kRound], wq[kRound];
      int offk[kRound], offq[kRound];
#pragma unroll
      for (int r = 0; r < kRound; ++r) {
        const int b = min(b0 + r * kPlanWaves, B - 1);
        wk[r] = load_window(p.pkv + size_t(b) * N, N, 0, lane, offk[r]);
        wq[r] = load_window(p.qv + size_t(b) * N, N, 0, lane, offq[r]);
      }
#pragma unroll
      for (int r = 0; r < kRound; ++r) {
        int ck = 0, cq = 0, lk = -1, lq = -1;
        scan_window(wk[r], 4 * lane, offk[r], N, ck, lk);
        scan_window(wq[r], 4 * lane, offq[r], N, cq, lq);
        if (b0 + r * kPlanWaves < B) put_info(b0 + r * kPlanWaves, ck, lk, cq, lq);
      }
    }
  } else {
#pragma unroll 1
    for (int b = wave; b < B; b += kPlanWaves) {
      int ck = 0, cq = 0, lk = -1, lq = -1;
#pragma unroll 1
      for (int base = 0; base < N + 3; base += 256) {
        int offk, offq;
        const uint32_t wk = load_window(p.pkv + size_t(b) * N, N, base, lane, offk);
        const uint32_t wq = load_window(p.qv + size_t(b) * N, N, base, lane, offq);
        scan_window(wk, base + 4 * lane, offk, N, ck, lk);
        scan_window(wq, base + 4 * lane, offq, N, cq, lq);
      }
      put_info(b, ck, lk, cq, lq);
    }
  }
  __syncthreads();

  // 2. index lists of the molecules that need them
#pragma unroll 1
  for (int b = wave; b < B; b += kPlanWaves) {
    const uint32_t w = s_info[b];
    if (!(w & kKPre)) write_ranks(p.pkv + size_t(b) * N, N, ws.kidx + size_t(b) * N, lane);
    if (!(w & kQPre)) write_ranks(p.qv + size_t(b) * N, N, ws.qidx + size_t(b) * N, lane);
  }

  // 3. item counts: small items per cost key, large items in total
  if (tid < B) {
    const MolItems m = mol_items(s_info[tid], H, p.cap, p.work_target);
    if (m.n > 0) {
      if (m.cls == 0) {
        if (m.splits > 1) atomicAdd(&s_cnt[m.key_full], H * (m.splits - 1));
        atomicAdd(&s_cnt[m.key_last], H);
        atomicAdd(&s_small, m.n);
      } else {
        atomicAdd(&s_large, m.n);
      }
    }
  }
  __syncthreads();
  if (tid < 64) {
    // first position of each key, keys in descending order (lane l: key 63 - l)
    const int v = s_cnt[kCostKeys - 1 - tid];
    int incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (tid >= off) incl += t;
    }
    s_cnt[kCostKeys - 1 - tid] = incl - v;
    if (tid == 0) {
      ws.hdr[0] = s_small;
      ws.hdr[1] = s_large;
    }
  }
  __syncthreads();

  // 4. items (one wave per molecule): a molecule's items are its query
  //    ranges, heads interleaved; small items go to the positions of their
  //    cost keys (longest first), large ones follow each other.  Lane r
  //    claims the positions of the wave's molecule of round r (64 rounds at
  //    a time), so one LDS atomic instruction serves them all.
#pragma unroll 1
  for (int b0 = wave; b0 < B; b0 += kPlanWaves * 64) {
    int bf = 0, bl = 0;
    {
      const int b = b0 + lane * kPlanWaves;
      if (b < B) {
        const MolItems m = mol_items(s_info[b], H, p.cap, p.work_target);
        const int n_full = H * (m.splits - 1);
        if (m.n > 0) {
          if (m.cls == 0) {
            if (n_full > 0) bf = atomicAdd(&s_cnt[m.key_full], n_full);
            bl = atomicAdd(&s_cnt[m.key_last], H) - n_full;
          } else {
            bf = bl = atomicAdd(&s_large_next, m.n);
          }
        }
      }
    }
#pragma unroll 1
    for (int r = 0; r < 64 && b0 + r * kPlanWaves < B; ++r) {
      const int b = b0 + r * kPlanWaves;
      const uint32_t w = s_info[b];
      const MolItems m = mol_items(w, H, p.cap, p.work_target);
      const int n_full = H * (m.splits - 1);
      const int base_full = __shfl(bf, r, 64);
      const int base_last = __shfl(bl, r, 64);
      const int nk = info_nk(w), nq = info_nq(w);
#pragma unroll 1
      for (int l = lane; l < m.n; l += 64) {
        const int sp = l / H, h = l - sp * H;
        const int4 item{b, h, (sp * m.qpi) | (min(nq, (sp + 1) * m.qpi) << 16),
                        int(uint32_t(nk) | (w & (kKPre | kQPre)))};
        const int pos = (l < n_full ? base_full : base_last) + l;
        if (m.cls == 0) ws.small_items[pos] = item;
        else ws.large_items[pos] = item;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// small / large kernels
// ---------------------------------------------------------------------------
// Copy 8 elements [e0, e0+8) of a row into registers.  These kernels run only
// with head_dim % 8 == 0 and 16-byte aligned rows, so a chunk lies either
// inside the row or entirely past its end (then it reads as zero).
template <typename T>
__device__ __forceinline__ typename Half<T>::Op8 load8(const T* row, int e0, int D) {
  typename Half<T>::Op8 v;
  if (e0 < D) {
    v = *reinterpret_cast<const typename Half<T>::Op8*>(row + e0);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = T(0.0f);
  }
  return v;
}

// A work item, read through the scalar cache (constant address space): the
// plan kernel wrote the list before this launch and nothing writes it during
// the launch.  A scalar load is waited for at the first use of the header,
// one item later, where a vector load would be waited for at once (its
// uniform value moves to scalar registers).
typedef __attribute__((address_space(4))) const int const_int;
__device__ __forceinline__ int4 load_item(const int4* items, int i) {
  const const_int* c = (const const_int*)items + 4 * i;
  return int4{c[0], c[1], c[2], c[3]};
}

// Position of the valid atom of rank r: the identity when the valid atoms are
// a prefix (idx == nullptr), else the plan's compacted list.
__device__ __forceinline__ int atom_at(const int* idx, int r) { return idx ? idx[r] : r; }

template <typename T>
__device__ __forceinline__ typename Half<T>::Op8 zero8() {
  typename Half<T>::Op8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = T(0.0f);
  return v;
}

// PART 0: the items of molecules with at most one key chunk (small items);
// PART 1: the items of larger molecules.
template <typename T, int DP, int NT, bool HAS_PV, int PART>
__device__ __forceinline__ void fast_body(const Params& p) {
  using Hf = Half<T>;
  using Op8 = typename Hf::Op8;
  using Op4 = typename Hf::Op4;
  using QOp = typename Hf::QOp;
  using K1T = typename Hf::K1T;
  using L = Layout<T, DP, NT>;
  constexpr int CH = L::CH;
  constexpr int KS = L::KS;
  constexpr int VS = L::VS;
  constexpr int WS = L::WS;
  constexpr int PW = L::PW;
  constexpr int NCH = DP / 32;        // 32-wide d chunks (GEMM1 K steps)
  constexpr int ND = DP / 16;         // 16-wide d tiles of GEMM2
  constexpr int NN = ND + 1;          // + the validity (denominator) tile
  constexpr int NPR = (NT + 1) / 2;   // 32-key K steps of GEMM2
  constexpr int CPR = DP / 8;         // 8-element chunks per padded row
  constexpr int RPP = kThreads / CPR; // rows per staging pass
  constexpr int RPT = (CH + RPP - 1) / RPP;
  constexpr int QPT = (kMaxQueriesPerItem + RPP - 1) / RPP;
  constexpr int NU = (NT * NCH + kWaves - 1) / kWaves;  // V1 tiles (16 keys x 32 columns) per wave
  static_assert(kThreads % CPR == 0, "a thread's 8-column chunk must be fixed across rows");

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  K1T* K1s = reinterpret_cast<K1T*>(smem + L::kK1);
  T* V2T = reinterpret_cast<T*>(smem + L::kV2T);
  unsigned char* VB = smem + L::kV2T;  // small items: GEMM2 B operands, 16 bytes per lane
  float* V1T = reinterpret_cast<float*>(smem + L::kV1T);
  using QT = typename Hf::QT;
  QT* Qs = reinterpret_cast<QT*>(smem + L::kQs);
  uint32_t* pvb = reinterpret_cast<uint32_t*>(smem + L::kPV);
  float* ab = reinterpret_cast<float*>(smem + L::kAB);
  float* red2 = reinterpret_cast<float*>(smem + L::kRed2);
  uint4* KA = reinterpret_cast<uint4*>(smem + L::kKA);
  float* red = reinterpret_cast<float*>(smem + L::kRed);
  float* qns = reinterpret_cast<float*>(smem + L::kQn);
  const int H = p.H, N = p.N, D = p.D;
  const Workspace& ws = p.ws;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const bool vec = p.vec_ok != 0;
  const T* gq = static_cast<const T*>(p.q);
  const T* gk1 = static_cast<const T*>(p.k1);
  const T* gk2 = static_cast<const T*>(p.k2);
  const T* gv1 = static_cast<const T*>(p.v1);
  const T* gv2 = static_cast<const T*>(p.v2);

  // XCD-aware logical workgroup id: blockIdx.x % 8 is the XCD, so give each
  // XCD a contiguous range of logical ids (gridDim.x is a multiple of 8).
  const int G = gridDim.x;
  const int wg = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);

  // Staging helpers -----------------------------------------------------------
  // K1s rows and V1T columns for compacted keys [j0, j0 + CH) (nkj valid),
  // V2T columns for keys [k0, k0 + CH) (nkk valid) when with_v; the column
  // maxima of |K1| go to red[] when with_max.
  auto stage_chunk = [&](const int* kidx, int bh, int j0, int nkj, int k0, int nkk, bool with_v, bool with_max) {
    const int c = tid % CPR;
    const int e0 = c * 8;
    Op8 a[RPT], v1v[RPT], v2v[RPT];
#pragma unroll
    for (int t = 0; t < RPT; ++t) {
      const int r = tid / CPR + t * RPP;
      a[t] = zero8<T>();
      v1v[t] = zero8<T>();
      v2v[t] = zero8<T>();
      if (r < nkj) {
        const size_t src = (size_t(bh) * N + atom_at(kidx, j0 + r)) * D;
        a[t] = load8<T>(gk1 + src, e0, D);
        if (with_v) v1v[t] = load8<T>(gv1 + src, e0, D);
      }
      if (with_v && r < nkk) v2v[t] = load8<T>(gv2 + (size_t(bh) * N + atom_at(kidx, k0 + r)) * D, e0, D);
    }
    float m1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) m1[e] = 0.0f;
#pragma unroll
    for (int t = 0; t < RPT; ++t) {
      const int r = tid / CPR + t * RPP;
      if (r < CH) {
        Hf::store_k1(K1s + r * L::K1S + e0, a[t]);
#pragma unroll
        for (int e = 0; e < 8; ++e) m1[e] = fmaxf(m1[e], fabsf(float(a[t][e])));
        if (with_v) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            V2T[(e0 + e) * VS + r] = v2v[t][e];
            V1T[(e0 + e) * WS + r] = float(v1v[t][e]);
          }
        }
      }
    }
    if (with_v) {
      // key validity row (DP) of V1T
      for (int u = tid; u < CH; u += kThreads) V1T[DP * WS + u] = u < nkj ? 1.0f : 0.0f;
    }
    if (with_max) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int off = CPR; off < 64; off <<= 1) m1[e] = fmaxf(m1[e], __shfl_xor(m1[e], off, 64));
      }
      if (lane < CPR) {
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wave * DP + e0 + e] = m1[e];
      }
    }
  };
  // pair-valid bits of the (j chunk, k chunk) block
  auto stage_pv = [&](const int* kidx, int b, int j0, int nkj, int k0, int nkk) {
    if constexpr (HAS_PV) {
      const uint8_t* gpv = p.pv + size_t(b) * N * N;
      for (int u = tid; u < CH * PW; u += kThreads) {
        const int jl = u / PW, w = u - jl * PW;
        uint32_t bits = 0;
        if (jl < nkj) {
          const uint8_t* prow = gpv + size_t(atom_at(kidx, j0 + jl)) * N;
          for (int t = 0; t < 32; ++t) {
            const int kl = w * 32 + t;
            if (kl < nkk && prow[atom_at(kidx, k0 + kl)] != 0) bits |= 1u << t;
          }
        }
        pvb[u] = bits;
      }
    }
  };
  // K2 rows [k0, k0 + nkk) of the compacted list as GEMM1 A operands
  auto load_ka = [&](Op8 (&ka)[NT][NCH], const int* kidx, int bh, int k0, int nkk) {
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      const int r = kt * 16 + r16;
      const int row = r < nkk ? atom_at(kidx, k0 + r) : 0;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        Op8 v = zero8<T>();
        if (r < nkk) v = load8<T>(gk2 + (size_t(bh) * N + row) * D, c * 32 + g * 8, D);
        ka[kt][c] = v;
      }
    }
  };
  // GEMM2 B operands: V2 columns d from V2T
  auto load_vb = [&](Op8 (&vb)[ND][NPR]) {
#pragma unroll
    for (int nt = 0; nt < ND; ++nt) {
#pragma unroll
      for (int pr = 0; pr < NPR; ++pr) {
        const T* vr = V2T + (nt * 16 + r16) * VS + 32 * pr + 4 * g;
        const Op4 lo4 = *reinterpret_cast<const Op4*>(vr);
        Op4 hi4;
        if (2 * pr + 1 < NT) {
          hi4 = *reinterpret_cast<const Op4*>(vr + 16);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) hi4[e] = T(0.0f);
        }
        vb[nt][pr] = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
  };
  // 0/1 selector B operands: sel[sh] picks columns 16 sh .. 16 sh + 15 of a
  // 32-column A tile (B[kk][n] = 1 iff kk == n + 16 sh).  Built per item
  // from an opaque zero so that they are not kept live through the query
  // loops.
  auto make_sel = [&](Op8 (&sel)[2]) {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
#pragma unroll
    for (int sh = 0; sh < 2; ++sh)
#pragma unroll
      for (int e = 0; e < 8; ++e) sel[sh][e] = T(8 * g + e + z == r16 + 16 * sh ? 1.0f : 0.0f);
  };
  // GEMM2 B operands of the denominator column: 1 in column 0 for full key
  // pairs; for the last pair of a chunk, 1 only at valid keys
  Op8 ones_full;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones_full[e] = T(r16 == 0 ? 1.0f : 0.0f);
  auto make_ones_edge = [&](int nkk) {
    const int last = (ceil_div(nkk, 16) - 1) >> 1;
    Op8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = 32 * last + (e < 4 ? 0 : 16) + 4 * g + (e & 3);
      v[e] = T((r16 == 0 && k < nkk) ? 1.0f : 0.0f);
    }
    return v;
  };
  // Row of a query: lane (g, r16) holds partial sums over its row group g of
  // the MFMA layout.  A reduce-scatter over the 4 groups (3 shuffles) leaves
  // lane (g, r16) with the full sum of d tile g (ND <= 4 tiles), and the
  // denominator partials of lanes (g, 0) are summed from 4 lane reads.
  auto write_row = [&](size_t row_off, float (&acc)[NN], float m) {
    static_assert(ND == 2 || ND == 4, "reduce-scatter shape");
    float x0, x1;
    {
      // groups {g, g ^ 2}: groups 0, 1 keep d tiles 0, 1; groups 2, 3 keep 2, 3
      const bool lo = g < 2;
      const float s0 = ND == 4 ? (lo ? acc[2 % ND] : acc[0]) : acc[0];
      const float s1 = ND == 4 ? (lo ? acc[3 % ND] : acc[1]) : acc[1];
      const float r0 = __shfl_xor(s0, 32, 64);
      const float r1 = __shfl_xor(s1, 32, 64);
      if constexpr (ND == 4) {
        x0 = (lo ? acc[0] : acc[2 % ND]) + r0;
        x1 = (lo ? acc[1] : acc[3 % ND]) + r1;
      } else {
        x0 = acc[0] + r0;
        x1 = acc[1] + r1;
      }
    }
    // groups {g, g ^ 1}: even groups keep x0, odd groups keep x1
    const bool odd = (g & 1) != 0;
    const float y = (odd ? x1 : x0) + __shfl_xor(odd ? x0 : x1, 16, 64);
    auto lane_val = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc[ND]), l)); };
    const float lsum = (lane_val(0) + lane_val(16)) + (lane_val(32) + lane_val(48));
    const bool has_mass = lsum > 0.0f;
    const float inv = has_mass ? 1.0f / lsum : 0.0f;
    const int nt = ND == 4 ? g : (g & 1);
    const int d = nt * 16 + r16;
    if ((ND == 4 || g < 2) && d < D) {
      const float o = y * inv;
      if (p.out) static_cast<T*>(p.out)[row_off * D + d] = T(o);
      if (p.out_f32) p.out_f32[row_off * D + d] = o;
    }
    if (lane == 0 && p.lse) p.lse[row_off] = has_mass ? (m + __log2f(lsum)) * kLn2 : 0.0f;
  };

  if constexpr (PART == 0) {
    // with an odd tile count the upper half of the last B operand (keys
    // 16 NT .. 16 NT + 15) is never written: zero
    if constexpr (NT % 2 == 1) {
      for (int u = tid; u < ND * 64; u += kThreads)
        *reinterpret_cast<uint2*>(VB + (((u / 64) * NPR + NPR - 1) * 64 + u % 64) * 16 + 8) = uint2{0u, 0u};
    }
    // The plan lists the items by estimated time, longest first.  Round r
    // gives item r G + w to workgroup w for even r and item r G + G - 1 - w
    // for odd r, so that each workgroup's long and short items pair up.
    const int n_items = ws.hdr[0];
    auto pos_of = [&](int r) { return r * G + ((r & 1) ? G - 1 - wg : wg); };
    int4 nxt = wg < n_items ? load_item(ws.small_items, wg) : int4{0, 0, 0, 0};
    for (int r = 0, item = wg; item < n_items; item = pos_of(++r)) {
      const int4 it = nxt;
      const int inext = pos_of(r + 1);
      if (inext < n_items) nxt = load_item(ws.small_items, inext);  // next header, one item ahead
      const int b = it.x, h = it.y, q0 = it.z & 0xffff, q1 = it.z >> 16, nk = it.w & 0xffff;
      const int bh = b * H + h;
      const int* kidx = (uint32_t(it.w) & kKPre) ? nullptr : ws.kidx + size_t(b) * N;
      const int* qidx = (uint32_t(it.w) & kQPre) ? nullptr : ws.qidx + size_t(b) * N;

      // ---- stage: one round of index loads, then one round of data loads ----
      const int njt = ceil_div(nk, 16);
      const int c8 = (tid % CPR) * 8;
      int jrow[RPT], qrow[QPT], krow[NT];
#pragma unroll
      for (int t = 0; t < RPT; ++t) {
        const int r = tid / CPR + t * RPP;
        jrow[t] = r < nk ? atom_at(kidx, r) : -1;
      }
#pragma unroll
      for (int t = 0; t < QPT; ++t) {
        const int r = tid / CPR + t * RPP;
        qrow[t] = r < q1 - q0 ? atom_at(qidx, q0 + r) : -1;
      }
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        const int r = kt * 16 + r16;
        krow[kt] = r < nk ? atom_at(kidx, r) : -1;
      }
      // K1 and query rows (one thread per 8 columns of a row); this wave's
      // share of the K2, V1 and V2 tiles (16 keys x 32 columns, tile
      // u = wave + kWaves i) in the MFMA A layout
      Op8 a[RPT], qv8[QPT];
      Op8 kaa[NU], va[NU], v1a[NU];
#pragma unroll
      for (int t = 0; t < RPT; ++t)
        a[t] = jrow[t] >= 0 ? load8<T>(gk1 + (size_t(bh) * N + jrow[t]) * D, c8, D) : zero8<T>();
#pragma unroll
      for (int t = 0; t < QPT; ++t)
        qv8[t] = qrow[t] >= 0 ? load8<T>(gq + (size_t(bh) * N + qrow[t]) * D, c8, D) : zero8<T>();
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = wave + kWaves * i, jt = u / NCH, c = u % NCH;
        const int key = jt * 16 + r16;
        const int row = jt < NT && key < nk ? atom_at(kidx, key) : -1;
        const size_t src = (size_t(bh) * N + row) * D;
        kaa[i] = row >= 0 ? load8<T>(gk2 + src, c * 32 + g * 8, D) : zero8<T>();
        v1a[i] = row >= 0 ? load8<T>(gv1 + src, c * 32 + g * 8, D) : zero8<T>();
        va[i] = row >= 0 ? load8<T>(gv2 + src, c * 32 + g * 8, D) : zero8<T>();
      }

      // LDS: query rows, K1 (and its column maxima), V1 transposed
#pragma unroll
      for (int t = 0; t < QPT; ++t) {
        const int r = tid / CPR + t * RPP;
        if (r < q1 - q0) Hf::store_q(Qs + r * KS + c8, qv8[t]);
        // |q'|_1 of the row (q' = q log2 e), reduced over its CPR chunk lanes
        float qn = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) qn += fabsf(float(qv8[t][e]));
#pragma unroll
        for (int off = 1; off < CPR; off <<= 1) qn += __shfl_xor(qn, off, 64);
        if (c8 == 0 && r < q1 - q0) qns[r] = qn * kLog2e;
      }
      {
        float m1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) m1[e] = 0.0f;
#pragma unroll
        for (int t = 0; t < RPT; ++t) {
          const int r = tid / CPR + t * RPP;
          if (r < CH) {
            Hf::store_k1(K1s + r * L::K1S + c8, a[t]);
#pragma unroll
            for (int e = 0; e < 8; ++e) m1[e] = fmaxf(m1[e], fabsf(float(a[t][e])));
          }
        }
        // the 8 lanes of a column chunk (lanes l ^ 8, l ^ 16, l ^ 32; 16 lanes
        // when CPR == 4) scatter the 8 column maxima among themselves
        int e1;
        float mx = reduce_scatter_max<8, 32>(m1, lane, e1);
#pragma unroll
        for (int off = 4; off >= CPR; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        red[wave * DP + c8 + e1] = mx;
      }
      if (tid < CH) V1T[DP * WS + tid] = tid < nk ? 1.0f : 0.0f;  // key validity row
      Op8 sel[2];
      make_sel(sel);
      // V1T[d][j] and the GEMM2 B operands of V2: an MFMA with a 0/1
      // selector B operand (exact) turns a 16-key x 32-column A tile into the
      // 16 x 16 C layout, lane (g, r16) holding keys 4g..4g+3 of column r16.
      // V1: one 16-byte store per lane into V1T.  V2: the bf16 keys
      // 4g..4g+3 of 16-key tile kt are half kt & 1 of operand (nt, kt / 2),
      // which holds keys 32 pr + 4g + 0..3 and 32 pr + 16 + 4g + 0..3
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = wave + kWaves * i, jt = u / NCH, c = u % NCH;
        if (jt < NT) {
#pragma unroll
          for (int sh = 0; sh < 2; ++sh) {
            const int nt = 2 * c + sh;
            if (jt < njt) {
              const mf_f32x4 t4 = Hf::mfma32(v1a[i], sel[sh], mf_f32x4{0.f, 0.f, 0.f, 0.f});
              *reinterpret_cast<float4*>(V1T + (nt * 16 + r16) * WS + jt * 16 + 4 * g) =
                  float4{t4[0], t4[1], t4[2], t4[3]};
            }
            const mf_f32x4 w4 = Hf::mfma32(va[i], sel[sh], mf_f32x4{0.f, 0.f, 0.f, 0.f});
            *reinterpret_cast<uint2*>(VB + ((nt * NPR + jt / 2) * 64 + lane) * 16 + (jt & 1) * 8) =
                uint2{Hf::pack(w4[0], w4[1]), Hf::pack(w4[2], w4[3])};
          }
        }
      }
      stage_pv(kidx, b, 0, nk, 0, nk);
      {
        // K2 operands to LDS, and this wave's column maxima of |K2|: per
        // column chunk over the wave's tiles, then a reduce-scatter over the
        // 16 key lanes (value v: column (v / 8) * 32 + 8 g + v % 8)
        constexpr int NV2 = NCH * 8;
        float mk[NV2];
#pragma unroll
        for (int v = 0; v < NV2; ++v) mk[v] = 0.0f;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
          const int u = wave + kWaves * i, c = u % NCH;
          if (u < NT * NCH) {
            KA[u * 64 + lane] = __builtin_bit_cast(uint4, kaa[i]);
#pragma unroll
            for (int cc = 0; cc < NCH; ++cc) {
              if (cc != c) continue;
#pragma unroll
              for (int e = 0; e < 8; ++e) mk[cc * 8 + e] = fmaxf(mk[cc * 8 + e], fabsf(float(kaa[i][e])));
            }
          }
        }
        int i2;
        float m2 = reduce_scatter_max<NV2, 8>(mk, lane, i2);
#pragma unroll
        for (int off = 16 / NV2 / 2; off >= 1; off >>= 1) m2 = fmaxf(m2, __shfl_xor(m2, off, 64));
        red2[wave * DP + (i2 / 8) * 32 + g * 8 + i2 % 8] = m2;
      }
      __syncthreads();
      Op8 vb[ND][NPR];
#pragma unroll
      for (int nt = 0; nt < ND; ++nt)
#pragma unroll
        for (int pr = 0; pr < NPR; ++pr)
          vb[nt][pr] = *reinterpret_cast<const Op8*>(VB + ((nt * NPR + pr) * 64 + lane) * 16);
      Op8 ka[NT][NCH];
#pragma unroll
      for (int kt = 0; kt < NT; ++kt)
#pragma unroll
        for (int c = 0; c < NCH; ++c) ka[kt][c] = __builtin_bit_cast(Op8, KA[(kt * NCH + c) * 64 + lane]);
      if (tid < DP) {
        float a0 = 0.0f, b0 = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          a0 = fmaxf(a0, red[w * DP + tid]);
          b0 = fmaxf(b0, red2[w * DP + tid]);
        }
        ab[tid] = a0 * b0;
      }
      __syncthreads();
      // sum_d |q'_d| m1_d m2_d <= |q'|_1 max_d (m1_d m2_d) = |q'|_1 M bounds |S| of a query
      const float mab = wave_max(lane < DP ? ab[lane] : 0.0f);
      const Op8 ones_edge = make_ones_edge(nk);

      if (njt == 0) {
        // valid queries of a molecule without keys: zero rows, lse 0
        for (int qs = q0 + wave; qs < q1; qs += kWaves) {
          float acc[NN];
#pragma unroll
          for (int nt = 0; nt < NN; ++nt) acc[nt] = 0.0f;
          write_row(size_t(bh) * N + atom_at(qidx, qs), acc, 0.0f);
        }
      }
      with_tiles<NT>(njt, [&](auto tiles) {
        constexpr int NKT = decltype(tiles)::value;
        for (int qs = q0 + wave; qs < q1; qs += kWaves) {
          const size_t row_off = size_t(bh) * N + atom_at(qidx, qs);
          QOp qo[NCH];
#pragma unroll
          for (int c = 0; c < NCH; ++c) Hf::load_q(Qs + (qs - q0) * KS + c * 32 + g * 8, qo[c]);
          const float ubound = qns[qs - q0] * mab;
          const bool fast = __builtin_amdgcn_readfirstlane(ubound <= p.bound_limit ? 1 : 0) != 0;
          float acc[NN];
#pragma unroll
          for (int nt = 0; nt < NN; ++nt) acc[nt] = 0.0f;
          float m = 0.0f;
          if (fast) {
            query_acc<T, DP, NT, NKT, HAS_PV, false>(K1s, V1T, pvb, ka, vb, ones_full, ones_edge, qo, nk, 0.0f, acc,
                                                     g, r16);
          } else {
            float mloc = -INFINITY;
#pragma unroll 1
            for (int jt = 0; jt < NKT; ++jt)
              mloc = fmaxf(mloc, jtile_max<T, DP, NT, NKT, HAS_PV>(K1s, pvb, ka, qo, jt, nk, nk, g, r16));
            m = wave_max(mloc);
            if (m != -INFINITY)
              query_acc<T, DP, NT, NKT, HAS_PV, true>(K1s, V1T, pvb, ka, vb, ones_full, ones_edge, qo, nk, m, acc, g,
                                                      r16);
          }
          write_row(row_off, acc, m);
        }
      });
      __syncthreads();
    }

  }
  if constexpr (PART == 1) {
    // ---- molecules larger than one chunk: one query per wave, chunk pairs ----
    const int n_items = ws.hdr[1];
    if (n_items > 0) __syncthreads();  // LDS of the last small item
    for (int item = wg; item < n_items; item += G) {
      const int4 it = ws.large_items[item];
      const int b = it.x, h = it.y, q0 = it.z & 0xffff, q1 = it.z >> 16, nk = it.w & 0xffff;
      const int bh = b * H + h;
      const int* kidx = (uint32_t(it.w) & kKPre) ? nullptr : ws.kidx + size_t(b) * N;
      const int* qidx = (uint32_t(it.w) & kQPre) ? nullptr : ws.qidx + size_t(b) * N;
      const int qs = q0 + wave;
      const bool has_q = qs < q1;
      const size_t row_off = size_t(bh) * N + (has_q ? atom_at(qidx, qs) : 0);
      QOp qo[NCH];
      if (has_q) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) Hf::prepare(load8<T>(gq + row_off * D, c * 32 + g * 8, D), qo[c]);
      }
      const int nch = ceil_div(nk, CH);
      float acc[NN];
#pragma unroll
      for (int nt = 0; nt < NN; ++nt) acc[nt] = 0.0f;
      float mloc = -INFINITY;
      float m = -INFINITY;
      for (int sweep = 0; sweep < 2; ++sweep) {
        for (int jc = 0; jc < nch; ++jc) {
          const int j0 = jc * CH, nkj = min(CH, nk - j0);
          for (int kc = 0; kc < nch; ++kc) {
            const int k0 = kc * CH, nkk = min(CH, nk - k0);
            stage_chunk(kidx, bh, j0, nkj, k0, nkk, sweep == 1, false);
            stage_pv(kidx, b, j0, nkj, k0, nkk);
            Op8 ka[NT][NCH];
            load_ka(ka, kidx, bh, k0, nkk);
            __syncthreads();
            const int njt = ceil_div(nkj, 16);
            if (sweep == 0) {
              if (has_q)
                for (int jt = 0; jt < njt; ++jt)
                  mloc = fmaxf(mloc, jtile_max<T, DP, NT, NT, HAS_PV>(K1s, pvb, ka, qo, jt, nkj, nkk, g, r16));
            } else {
              Op8 vb[ND][NPR];
              load_vb(vb);
              const Op8 ones_edge = make_ones_edge(NT * 16);
              if (has_q && m != -INFINITY)
                for (int jt = 0; jt < njt; ++jt)
                  jtile_acc<T, DP, NT, NT, HAS_PV, true>(K1s, V1T, pvb, ka, vb, ones_full, ones_edge, qo, jt, nkj,
                                                         nkk, m, acc, g, r16);
            }
            __syncthreads();
          }
        }
        if (sweep == 0) m = wave_max(mloc);
      }
      if (has_q) write_row(row_off, acc, m == -INFINITY ? 0.0f : m);
    }
  }
}

// MODE 0: small items only (every molecule fits one key chunk); MODE 1:
// small items, then the larger molecules.
template <typename T, int DP, int NT, bool HAS_PV, int MODE>
__global__ void __launch_bounds__(kThreads, 2) simplicial_fast_kernel(Params p) {
  fast_body<T, DP, NT, HAS_PV, 0>(p);
  if constexpr (MODE == 1) fast_body<T, DP, NT, HAS_PV, 1>(p);
}

template <typename T, int DP, int NT, bool HAS_PV, int MODE>
int launch_main(const Params& prm, int grid, hipStream_t stream) {
  auto kern = simplicial_fast_kernel<T, DP, NT, HAS_PV, MODE>;
  const size_t lds = Layout<T, DP, NT>::kFixed;
  const int st = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), int(lds));
  if (st != MF_OK) return st;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, stream, prm);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

template <typename T, int DP, int NT, bool HAS_PV>
int launch_all(const Params& prm, int num_cus, hipStream_t stream) {
  // workgroup 0 plans, the others zero the rows of padded queries
  hipLaunchKernelGGL(simplicial_plan_kernel, dim3(std::max(2, num_cus)), dim3(kPlanThreads), 0, stream, prm);
  MF_HIP_CHECK(hipGetLastError());
  const int grid = num_cus * 2;  // a multiple of 8 (the XCD count)
  if (prm.N <= prm.cap) return launch_main<T, DP, NT, HAS_PV, 0>(prm, grid, stream);
  return launch_main<T, DP, NT, HAS_PV, 1>(prm, grid, stream);
}

}  // namespace sfast

// Key capacity of one chunk of the fast kernels for a head dim, or 0 when
// they do not serve this head dim.
int simplicial_fast_capacity(int head_dim) {
  if (head_dim <= 32) return 16 * 6;
  if (head_dim <= 64) return 16 * 5;
  return 0;
}

size_t simplicial_fast_workspace_bytes(int batch, int heads, int tokens) {
  const int b = std::min(batch, sfast::kMaxBatch);
  return sfast::workspace_bytes(b, heads, tokens);
}

// One set of launches over a[0..batch), batch <= sfast::kMaxBatch.
int simplicial_fast_launch(const mf_simplicial_fwd_args* a, void* workspace, int num_cus, hipStream_t stream) {
  using namespace sfast;
  if (a->batch > kMaxBatch) return fail(MF_ERR_INVALID_ARGUMENT, "simplicial fast launch: batch slice too large");
  Params prm{};
  prm.q = a->q; prm.k1 = a->k1; prm.v1 = a->v1; prm.k2 = a->k2; prm.v2 = a->v2;
  prm.qv = a->query_valid; prm.pkv = a->pair_key_valid; prm.pv = a->pair_valid;
  prm.out = a->out; prm.out_f32 = a->out_f32; prm.lse = a->lse;
  prm.B = a->batch; prm.H = a->heads; prm.N = a->tokens; prm.D = a->head_dim;
  prm.ws = carve_workspace(workspace, a->batch, a->heads, a->tokens);
  prm.cap = simplicial_fast_capacity(a->head_dim);
  prm.work_target = 128 * 1024;
  prm.bound_limit = a->dtype == MF_DTYPE_BF16 ? 60.0f : 14.0f;
  bool vec = (a->head_dim * 2) % 16 == 0;
  for (const void* ptr : {a->q, a->k1, a->v1, a->k2, a->v2, static_cast<const void*>(a->out)})
    vec = vec && (reinterpret_cast<uintptr_t>(ptr) % 16 == 0);
  if (a->out_f32) vec = vec && (reinterpret_cast<uintptr_t>(a->out_f32) % 16 == 0);
  prm.vec_ok = vec ? 1 : 0;
  const bool pv = a->pair_valid != nullptr;
  const bool bf = a->dtype == MF_DTYPE_BF16;
  if (a->head_dim <= 32) {
    if (bf) return pv ? launch_all<__bf16, 32, 6, true>(prm, num_cus, stream) : launch_all<__bf16, 32, 6, false>(prm, num_cus, stream);
    return pv ? launch_all<_Float16, 32, 6, true>(prm, num_cus, stream) : launch_all<_Float16, 32, 6, false>(prm, num_cus, stream);
  }
  if (bf) return pv ? launch_all<__bf16, 64, 5, true>(prm, num_cus, stream) : launch_all<__bf16, 64, 5, false>(prm, num_cus, stream);
  return pv ? launch_all<_Float16, 64, 5, true>(prm, num_cus, stream) : launch_all<_Float16, 64, 5, false>(prm, num_cus, stream);
}

}  // namespace mf

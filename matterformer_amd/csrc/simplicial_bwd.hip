// 2-simplicial attention backward for gfx950 (CDNA4), deterministic.
//
// Math (the gradient of simplicial_attention.py:206-344; the same quantities
// as triton_simplicial_attention.py:332-782, which sums them with atomics):
//   P_ijk  = exp(S_ijk - lse_i) on valid pairs, S_ijk = sum_d q_id k1_jd k2_kd
//            (+ gate_i (u_ij + v_ik + w_jk))
//   dP_ijk = sum_d go_id v1_jd v2_kd,   dS_ijk = P_ijk (dP_ijk - go_i . out_i)
//   dq_i   = sum_jk dS k1_j (.) k2_k     dk1_j = sum_i q_i (.) sum_k dS k2_k
//   dk2_k  = sum_i q_i (.) sum_j dS k1_j dv1_j = sum_i go_i (.) sum_k P v2_k
//   dv2_k  = sum_i go_i (.) sum_j P v1_j
//   du_ij  = gate_i sum_k dS   dv_ik = gate_i sum_j dS   dw_jk = sum_i gate_i dS
//   dgate_i = sum_jk dS (u_ij + v_ik + w_jk)
//
// Ownership instead of atomics.  Every gradient row belongs to one index:
// dq, du, dv, dgate to the query i; dk1, dv1, dw to the key j; dk2, dv2 to
// the key k.  The three "roles" are one trilinear pattern with the operands
// permuted (S_ijk is symmetric under q <-> k1 <-> k2 with the masks moved):
//
//   role outer o rows r cols c  S = C_S . (oS (.) R_S)      dP = C_P . (oP (.) R_P)   value paths
//   Q    i       j      k       K2 . (q_i (.) K1[j])       V2 . (go_i (.) V1[j])    dS: K1[j] (.) K2 -> dq_i
//   J    j       i      k       K2 . (k1_j (.) Q[i])       V2 . (v1_j (.) GO[i])    dS: Q (.) K2 -> dk1_j, P: GO (.) V2 -> dv1_j
//   K    k       i      j       K1 . (k2_k (.) Q[i])       V1 . (v2_k (.) GO[i])    dS: Q (.) K1 -> dk2_k, P: GO (.) V1 -> dv2_k
//
// One launch for the three roles, OB workgroups per (b, h) and role; workgroup ob takes the outer indices
// (it OB + ob) kWaves + wave, one per wave and iteration it, so every
// gradient element is written by one wave after sums in a fixed order: no
// atomics, bitwise reproducible.  OB is sized on the host to fill the device
// (no workgroup lands wholly past the valid atoms of small molecules); the
// key columns, staged per 64-column block, stay in LDS across iterations when
// a molecule has at most 64 valid keys.
//
// Per wave: for each 64-column block (keys, staged in LDS as C_S and C_P,
// shared by the waves) and each 16-row tile (rows read from L2, 4
// consecutive d per lane):
//   GEMM1   S^T[c][r]  = sum_d C_S[c][d] (oS (.) R_S[r])[d]   fp32 MFMA 16x16x4
//   GEMM1'  dP^T[c][r] = sum_d C_P[c][d] (oP (.) R_P[r])[d]
//   P = exp2(S2 - lse2) (log2 e folded into oS), dS = P (dP - delta)
//   GEMM2   C2a[d][r] += sum_c C_S[c][d] dS[r][c]  (and C2b with C_P and P)
//   out_o[d] += R[r][d] C2[d][r]   (fp32, the row values already in registers)
// The accumulator layout of GEMM1 (lane = row r, 4 consecutive columns per
// lane group) is the B-operand layout GEMM2 needs, as in the forward.
//
// Two arithmetic paths share everything but the two GEMMs:
//   fp32 inputs: fp32 MFMA 16x16x4, all products and sums fp32.  The K index
//     is mapped to d = 16 t + 4 g + e so that each lane reads 4 consecutive
//     d of a row (one 16-byte load) for 4 MFMA steps.
//   bf16 inputs: bf16 MFMA 16x16x32 with fp32 accumulation, at the
//     reference backward's precision (triton_simplicial_attention.py:546-551
//     rounds only the score products q (.) k to the input type; its dP and
//     dS / P contractions, :611-645, are fp32).  Columns and rows are staged
//     as bf16 (exact).  The GEMM1 B operand is the fp32 product oS (.) R
//     rounded to bf16 for S, and carried as bf16 hi + lo (x = hi + lo to
//     about 16 bits, two MFMAs) for dP, whose difference dP - delta cancels
//     when one pair dominates the softmax; 8 consecutive d = 32 s + 8 g .. +7
//     per lane.  GEMM2 takes dS and P rounded once to bf16 (their sums over
//     the columns carry no cancellation) as its B operand
//     straight from the GEMM1 accumulators of two column tiles, and
//     C_S^T / C_P^T as its A operand through transposed LDS reads
//     (ds_read_b64_tr_b16) of the row-major columns.  Softmax, dS and every
//     sum stay fp32.  Lane (g, r16) holds d = 32 (t >> 1) + 8 g + 4 (t & 1)
//     + e of tile t: the same d for its GEMM1 operands, its GEMM2 outputs
//     and its row values.
//   fp16 inputs take the fp32 path (fp16 columns are not exact in bf16).
//
// Low-rank angle and message terms (LR instantiations, fp32 path, 4 waves):
// every pair (i, j, k) a lane evaluates gains the rank dot products of its
// query's factors, A = sum_r AL[i,j,r] AR[i,k,r] into S and
// M = sum_r dc_ir ML[i,j,r] MR[i,k,r] into dP (dc_ir = basis[h,r] . go_i,
// written to the workspace by a pre-pass).  One factor of each dot depends
// on the lane's row and the outer index only and is read once per rank
// chunk; the other is read per column:
//   role Q (i = o):  row AL[o,j=row], ML[o,row];  column AR[o,k=col], MR[o,col]
//   role J (j = o):  row AL[i=row,o], ML[row,o];  column AR[row,k=col], MR[row,col]
//   role K (k = o):  row AR[i=row,o], MR[row,o];  column AL[row,j=col], ML[row,col]
// All gradients of these terms are indexed by the query i, so ownership
// still decides who writes them: role Q sums dangle_left[o,row] and
// dmessage_left[o,row] over its columns, role K dangle_right[row,o] and
// dmessage_right[row,o]; each wave adds its column blocks' sums in order.
// Role Q also forms sum_jk P ML MR per query (per-row partials in LDS) for
// dmessage_basis, which a post-pass reduces over the batch in a fixed order.
#include <algorithm>
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace sbwd {

constexpr int kRoleQ = 0;
constexpr int kRoleJ = 1;
constexpr int kRoleK = 2;
constexpr int kCols = 64;  // staged key columns per block

template <int DP, bool M16, bool LR = false>
struct Shape {
  // fp32: D = 128 needs the whole register file per wave, as do the rank
  // terms (LR).  16-bit: 4 waves at about 240 VGPRs put two workgroups on
  // each CU, so that one's global loads overlap the other's arithmetic.
  static constexpr int kWaves = (M16 || DP >= 128 || LR) ? 4 : 8;
  static constexpr int kMinBlocks = (M16 && DP < 128) ? 2 : 1;  // workgroups per CU the registers must allow
  static constexpr int kThreads = kWaves * 64;
  static constexpr int NT = DP / 16;   // 16-wide d tiles
  static constexpr int D4 = DP + 4;    // LDS row stride (floats) of the staged fp32 columns
  static constexpr int KS = DP + 8;    // LDS row stride (bf16) of the staged 16-bit columns
};

// First d of the 4 that lane group g holds in d tile t (see the header).
template <bool M16>
__device__ __forceinline__ int dof(int t, int g) {
  return M16 ? 32 * (t >> 1) + 8 * g + 4 * (t & 1) : 16 * t + 4 * g;
}

__device__ __forceinline__ mf_bf16x8 pack_bf16(const float4& lo, const float4& hi) {
  mf_bf16x8 r;
  r[0] = __bf16(lo.x); r[1] = __bf16(lo.y); r[2] = __bf16(lo.z); r[3] = __bf16(lo.w);
  r[4] = __bf16(hi.x); r[5] = __bf16(hi.y); r[6] = __bf16(hi.z); r[7] = __bf16(hi.w);
  return r;
}

__device__ __forceinline__ float4 bf16_lo(const mf_bf16x8& v) {
  return float4{float(v[0]), float(v[1]), float(v[2]), float(v[3])};
}
__device__ __forceinline__ float4 bf16_hi(const mf_bf16x8& v) {
  return float4{float(v[4]), float(v[5]), float(v[6]), float(v[7])};
}

__device__ __forceinline__ float4 mul4(const float4& a, const float4& b) {
  return float4{a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w};
}



struct Params {
  const void* q;
  const void* k1;
  const void* v1;
  const void* k2;
  const void* v2;
  const void* go;
  const float* out;
  const float* lse;
  const uint8_t* qv;
  const uint8_t* pkv;
  const uint8_t* pv;
  const void* u;
  const void* vb;
  const void* w;
  const void* gate;
  int bias_dtype;
  void* dq;      // gradients, fp32 or (gout16) bf16
  void* dk1;
  void* dv1;
  void* dk2;
  void* dv2;
  int gout16;
  void* du;      // bias gradients, fp32 or (gout16) bf16
  void* dvb;
  void* dw;
  void* dgate;
  int B, H, N, D;
  int dtype, gdtype;
  int NP;       // N rounded up to 64: LDS list capacity
  int OB;       // workgroups per (b, h, role)
  int vec;      // q/k/v/go/out rows 4-element loads are aligned (D % 4 == 0, aligned bases)
  const int* served;  // [B] nonzero: the pair kernel computed this molecule's gradients (or NULL)
  const int* unserved;  // the number of molecules the pair kernel left over (with `served`)
  int blocks;         // 3 B H OB work blocks; the grid may be smaller and loop over them
  int served_lds;     // byte offset of the LDS copy of `served` (after the role's layout)
  // low-rank terms (LR instantiations): factors [B*H, N, N, R] fp32, gates [B*H, N], basis [H, Rm, D]
  const float* al;
  const float* ar;
  const float* ag;
  const float* ml;
  const float* mr;
  const float* mb;
  int Ra, Rm, RmP;      // ranks; Rm rounded up to 4
  float a_scale, m_scale;
  int lr_vec;           // rank rows are 16-byte aligned (R % 4 == 0, aligned bases): float4 reads
  float* dal;
  float* dar;
  float* dag;
  float* dml;
  float* dmr;
  float* dc;            // workspace [B*H, N, Rm]: basis[h] . go_i (message)
  float* coeff;         // workspace [B*H, N, Rm]: sum_jk P ML MR of each valid query (message)
};

// LDS layout (bytes), shared by host sizing and device carving.
template <int DP, bool M16, bool LR = false>
struct Lay {
  // staged tiles: fp32 C_S, C_P (64 columns); 16-bit: bf16 C_S, C_P and R_S, R_P (64 rows)
  static size_t __host__ __device__ cols() {
    return M16 ? size_t(4) * kCols * Shape<DP, M16>::KS * 2 : size_t(2) * kCols * Shape<DP, M16>::D4 * 4;
  }
  static size_t __host__ __device__ bytes(int NP, bool has_pv, bool has_bias, int RmP = 0) {
    size_t s = cols();
    s += size_t(NP) * 4 * 4;                                  // kidx, qidx, delta, lse2
    if (has_pv) s += size_t(NP) * 2 * 4;                      // 64 column bits per row
    if (has_bias) s += size_t(Shape<DP, M16, LR>::kWaves) * (NP + kCols) * 4;  // per-wave row / column sums
    s += 16;                                                  // counts
    s += size_t(Shape<DP, M16, LR>::kWaves) * 16 * RmP * 4;   // LR: per-wave, per-row sum_jk P ML MR partials
    return s;
  }
};

__device__ __forceinline__ float ld1(const void* p, size_t i, int dt) {
  if (dt == MF_DTYPE_F32) return static_cast<const float*>(p)[i];
  if (dt == MF_DTYPE_BF16) return static_cast<float>(static_cast<const __bf16*>(p)[i]);
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}

// Elements d0..d0+3 of row `row` (length D) of a [.., D] tensor, 0 past D.
__device__ __forceinline__ float4 ld4(const void* p, size_t row, int d0, int D, int dt, bool vec) {
  const size_t base = row * size_t(D) + d0;
  if (vec && d0 + 3 < D) {
    if (dt == MF_DTYPE_F32) return *reinterpret_cast<const float4*>(static_cast<const float*>(p) + base);
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + base);
    float4 r;
    if (dt == MF_DTYPE_BF16) {
      r.x = __uint_as_float(raw.x << 16);
      r.y = __uint_as_float(raw.x & 0xffff0000u);
      r.z = __uint_as_float(raw.y << 16);
      r.w = __uint_as_float(raw.y & 0xffff0000u);
    } else {
      const _Float16* h = reinterpret_cast<const _Float16*>(&raw);
      r.x = float(h[0]); r.y = float(h[1]); r.z = float(h[2]); r.w = float(h[3]);
    }
    return r;
  }
  float4 r;
  r.x = d0 < D ? ld1(p, base, dt) : 0.0f;
  r.y = d0 + 1 < D ? ld1(p, base + 1, dt) : 0.0f;
  r.z = d0 + 2 < D ? ld1(p, base + 2, dt) : 0.0f;
  r.w = d0 + 3 < D ? ld1(p, base + 3, dt) : 0.0f;
  return r;
}

// One gradient element, fp32 or rounded to bf16.
__device__ __forceinline__ void store_grad(void* base, size_t i, float v, int bf16) {
  if (bf16) static_cast<__bf16*>(base)[i] = __bf16(v);
  else static_cast<float*>(base)[i] = v;
}

__device__ __forceinline__ float f4(const float4& v, int e) {
  return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

// Compact the valid positions of a byte mask row into dst; returns the count.
__device__ __forceinline__ int compact(const uint8_t* m, int N, int* dst, int lane) {
  int count = 0;
  for (int base = 0; base < N; base += 64) {
    const int t = base + lane;
    const bool v = t < N && m[t] != 0;
    const unsigned long long bal = __ballot(v);
    if (v) dst[count + __popcll(bal & ((1ull << lane) - 1ull))] = t;
    count += __popcll(bal);
  }
  return count;
}

// Elements r0 .. r0 + 3 of a rank row (rem = R - r0 >= 1 of them valid, the
// rest 0); one 16-byte read when the rows are aligned and R % 4 == 0.
__device__ __forceinline__ float4 ld_r4(const float* p, int rem, int vec) {
  if (vec) return *reinterpret_cast<const float4*>(p);
  float4 r = float4{p[0], 0.f, 0.f, 0.f};
  if (rem > 1) r.y = p[1];
  if (rem > 2) r.z = p[2];
  if (rem > 3) r.w = p[3];
  return r;
}

// DPP moves within 16-lane rows (VALU, no LDS): quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __uint_as_float(uint32_t(__builtin_amdgcn_update_dpp(0, int(__float_as_uint(v)), CTRL, 0xf, 0xf, false)));
}

// Sum over each 16-lane row, in every lane of the row (pairs, quads, halves, rows).
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<0xb1>(x);
  x += dpp_f<0x4e>(x);
  x += dpp_f<0x141>(x);
  return x + dpp_f<0x140>(x);
}

// Sum over the four 16-lane rows, (r0 + r2) + (r1 + r3) in every lane: the gfx950 lane swaps.
__device__ __forceinline__ float rows4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// x + its partners in the other three 16-lane groups (lanes l ^ 16, l ^ 32), in a fixed order
__device__ __forceinline__ float4 sum_groups4(float4 v) {
  v.x += __shfl_xor(v.x, 16, 64); v.y += __shfl_xor(v.y, 16, 64);
  v.z += __shfl_xor(v.z, 16, 64); v.w += __shfl_xor(v.w, 16, 64);
  v.x += __shfl_xor(v.x, 32, 64); v.y += __shfl_xor(v.y, 32, 64);
  v.z += __shfl_xor(v.z, 32, 64); v.w += __shfl_xor(v.w, 32, 64);
  return v;
}

template <int DP, int ROLE, bool M16, bool BIAS, bool LR>
__device__ __forceinline__ void run_role(const Params& p, unsigned char* smem, int bh, int ob) {
  using S = Shape<DP, M16, LR>;
  constexpr int kWaves = S::kWaves;
  constexpr int kThreads = S::kThreads;
  constexpr int NT = S::NT;
  constexpr int D4 = S::D4;
  constexpr int KS = S::KS;
  const int N = p.N, D = p.D, NP = p.NP;
  const int b = bh / p.H;
  const bool has_pv = p.pv != nullptr;
  constexpr bool has_bias = BIAS;
  const bool vec = p.vec != 0;

  float* CS = reinterpret_cast<float*>(smem);  // fp32 columns (fp32 path)
  float* CP = CS + kCols * D4;
  __bf16* CS16 = reinterpret_cast<__bf16*>(smem);  // bf16 columns and rows (16-bit path)
  __bf16* CP16 = CS16 + kCols * KS;
  __bf16* RS16 = CP16 + kCols * KS;
  __bf16* RP16 = RS16 + kCols * KS;
  int* kidx = reinterpret_cast<int*>(smem + Lay<DP, M16>::cols());
  int* qidx = kidx + NP;
  float* delta = reinterpret_cast<float*>(qidx + NP);  // go . out of each valid query (roles J, K)
  float* lse2q = delta + NP;                           // lse log2 e of each valid query (roles J, K)
  uint32_t* pvb = reinterpret_cast<uint32_t*>(lse2q + NP);
  float* wrow = reinterpret_cast<float*>(pvb + (has_pv ? 2 * NP : 0));
  float* wcol = wrow + (has_bias ? kWaves * NP : 0);
  int* counts = reinterpret_cast<int*>(wcol + (has_bias ? kWaves * kCols : 0));
  float* coeffL = reinterpret_cast<float*>(counts + 4);  // LR: [kWaves][16][RmP] per-row sum_jk P ML MR partials

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;
  const int r16 = lane & 15;

  // ---- compacted key and query lists of molecule b ----
  if (wave == 0) {
    const int nk = compact(p.pkv + size_t(b) * N, N, kidx, lane);
    if (lane == 0) counts[0] = nk;
  } else if (wave == 1) {
    const int nq = compact(p.qv + size_t(b) * N, N, qidx, lane);
    if (lane == 0) counts[1] = nq;
  }
  __syncthreads();
  const int nk = counts[0], nq = counts[1];
  const int n_outer = ROLE == kRoleQ ? nq : nk;
  const int n_rows = ROLE == kRoleQ ? nk : nq;
  if (ob * kWaves >= n_outer || nk == 0 || nq == 0) return;  // uniform over the workgroup
  const int* outer_list = ROLE == kRoleQ ? qidx : kidx;
  const int* row_list = ROLE == kRoleQ ? kidx : qidx;

  // tensors of each role (rows of [B*H, N, D])
  const void* t_os = ROLE == kRoleQ ? p.q : (ROLE == kRoleJ ? p.k1 : p.k2);   // outer, S side
  const void* t_op = ROLE == kRoleQ ? p.go : (ROLE == kRoleJ ? p.v1 : p.v2);  // outer, dP side
  const int dt_op = ROLE == kRoleQ ? p.gdtype : p.dtype;
  const void* t_rs = ROLE == kRoleQ ? p.k1 : p.q;    // rows, S side
  const void* t_rp = ROLE == kRoleQ ? p.v1 : p.go;   // rows, dP side
  const int dt_rp = ROLE == kRoleQ ? p.dtype : p.gdtype;
  const void* t_cs = ROLE == kRoleK ? p.k1 : p.k2;   // columns, S side
  const void* t_cp = ROLE == kRoleK ? p.v1 : p.v2;   // columns, dP side
  const size_t rbase = size_t(bh) * N;               // first row of (b, h)

  // ---- delta_i = go_i . out_i and lse_i log2 e of every valid query (rows of roles J / K) ----
  // CH consecutive lanes share a query, 8 d each, summed in a fixed order.
  if constexpr (ROLE != kRoleQ) {
    constexpr int CH = DP / 8;
    for (int u0 = 0; u0 < nq * CH; u0 += kThreads) {
      const int u = u0 + tid;
      const int r = u / CH;
      const int d0 = (u - r * CH) * 8;
      const bool ok = u < nq * CH;
      float s = 0.0f;
      if (ok) {
        const size_t row = rbase + qidx[r];
        const float4 g0 = ld4(p.go, row, d0, D, p.gdtype, vec), g1 = ld4(p.go, row, d0 + 4, D, p.gdtype, vec);
        const float4 o0 = ld4(p.out, row, d0, D, MF_DTYPE_F32, vec);
        const float4 o1 = ld4(p.out, row, d0 + 4, D, MF_DTYPE_F32, vec);
        s = g0.x * o0.x;
        s = fmaf(g0.y, o0.y, s); s = fmaf(g0.z, o0.z, s); s = fmaf(g0.w, o0.w, s);
        s = fmaf(g1.x, o1.x, s); s = fmaf(g1.y, o1.y, s); s = fmaf(g1.z, o1.z, s); s = fmaf(g1.w, o1.w, s);
      }
#pragma unroll
      for (int off = 1; off < CH; off <<= 1) s += __shfl_xor(s, off, 64);
      if (ok && d0 == 0) {
        delta[r] = s;
        lse2q[r] = p.lse[rbase + qidx[r]] * kLog2e;
      }
    }
  }

  // ---- the workgroup's outer indices: (it * OB + ob) * kWaves + wave, it = 0 .. n_it - 1 ----
  // With one column block (nk <= kCols) the block is staged once for all iterations.
  const int n_it = (n_outer - ob * kWaves + kWaves * p.OB - 1) / (kWaves * p.OB);
  for (int it = 0; it < n_it; ++it) {
  const int ol = (it * p.OB + ob) * kWaves + wave;
  const bool active = ol < n_outer;
  const int oo = active ? outer_list[ol] : 0;
  const size_t orow = rbase + oo;
  float4 oS[NT], oP[NT];  // outer vectors at d = dof(t, g) + e (oS carries log2 e)
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    oS[t] = float4{0.f, 0.f, 0.f, 0.f};
    oP[t] = float4{0.f, 0.f, 0.f, 0.f};
    if (active) {
      const float4 a = ld4(t_os, orow, dof<M16>(t, g), D, p.dtype, vec);
      oS[t] = float4{a.x * kLog2e, a.y * kLog2e, a.z * kLog2e, a.w * kLog2e};
      oP[t] = ld4(t_op, orow, dof<M16>(t, g), D, dt_op, vec);
    }
  }
  float lse2_o = 0.0f, delta_o = 0.0f, gate_o = 0.0f;
  if constexpr (ROLE == kRoleQ) {
    if (active) {
      lse2_o = p.lse[orow] * kLog2e;
      float s = 0.0f;
      for (int d = lane; d < D; d += 64) s += ld1(p.go, orow * D + d, p.gdtype) * p.out[orow * D + d];
      delta_o = wave_sum(s);
      if (has_bias) gate_o = ld1(p.gate, orow, p.bias_dtype);
    }
  }

  float acc_a[NT][4], acc_b[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc_a[t][r] = 0.0f;
      acc_b[t][r] = 0.0f;
    }
  float gacc = 0.0f;  // role Q: dgate partial
  float gacc_a = 0.0f;  // role Q (LR): dangle_gate partial
  if constexpr (LR && ROLE == kRoleQ) {
    if (p.ml && p.coeff)
      for (int u = lane; u < 16 * p.RmP; u += 64) coeffL[wave * 16 * p.RmP + u] = 0.0f;
  }

  const int ncb = (nk + kCols - 1) / kCols;
  const int nrb = M16 ? (n_rows + kCols - 1) / kCols : 1;  // 16-bit: rows staged in 64-row blocks
  for (int cbi = 0; cbi < ncb; ++cbi) {
  const int cb0 = cbi * kCols;
  const int ncols = min(kCols, nk - cb0);
  for (int rbi = 0; rbi < nrb; ++rbi) {
    const int rb0 = rbi * kCols;
    const bool stage = rbi == 0 && (it == 0 || ncb > 1);             // the column block
    const bool stage_r = M16 && (nrb > 1 || (it == 0 && cbi == 0));  // the row block
    if (stage || stage_r) __syncthreads();  // the previous contents' LDS reads are done
    // stage the column block (fp32 or bf16, zero past nk and past D)
    if (!stage) {
    } else if constexpr (M16) {
      constexpr int CPR = DP / 8;  // 8-element chunks per row
      for (int u = tid; u < kCols * CPR; u += kThreads) {
        const int c = u / CPR;
        const int d0 = (u - c * CPR) * 8;
        const float4 z = float4{0.f, 0.f, 0.f, 0.f};
        mf_bf16x8 a = pack_bf16(z, z), bb = a;
        if (cb0 + c < nk) {
          const size_t row = rbase + kidx[cb0 + c];
          a = pack_bf16(ld4(t_cs, row, d0, D, p.dtype, vec), ld4(t_cs, row, d0 + 4, D, p.dtype, vec));
          bb = pack_bf16(ld4(t_cp, row, d0, D, p.dtype, vec), ld4(t_cp, row, d0 + 4, D, p.dtype, vec));
        }
        *reinterpret_cast<mf_bf16x8*>(CS16 + c * KS + d0) = a;
        *reinterpret_cast<mf_bf16x8*>(CP16 + c * KS + d0) = bb;
      }
    } else {
      constexpr int CPR = DP / 4;  // float4 chunks per row
      for (int u = tid; u < kCols * CPR; u += kThreads) {
        const int c = u / CPR;
        const int d0 = (u - c * CPR) * 4;
        float4 a = float4{0.f, 0.f, 0.f, 0.f}, bb = a;
        if (cb0 + c < nk) {
          const size_t row = rbase + kidx[cb0 + c];
          a = ld4(t_cs, row, d0, D, p.dtype, vec);
          bb = ld4(t_cp, row, d0, D, p.dtype, vec);
        }
        *reinterpret_cast<float4*>(CS + c * D4 + d0) = a;
        *reinterpret_cast<float4*>(CP + c * D4 + d0) = bb;
      }
    }
    if (stage && has_pv) {
      // bits of the block's 64 columns for every compacted key x:
      //   roles Q, J: pair_valid[x][column]; role K: pair_valid[column][x]
      const uint8_t* pvm = p.pv + size_t(b) * N * N;
      for (int u = tid; u < nk * 2; u += kThreads) {
        const int x = u >> 1;
        const int wd = u & 1;
        uint32_t bits = 0;
        for (int t = 0; t < 32; ++t) {
          const int c = cb0 + 32 * wd + t;
          if (c < nk) {
            const size_t idx = ROLE == kRoleK ? size_t(kidx[c]) * N + kidx[x] : size_t(kidx[x]) * N + kidx[c];
            if (pvm[idx]) bits |= 1u << t;
          }
        }
        pvb[2 * x + wd] = bits;
      }
    }
    if constexpr (M16) {
      // stage the row block (bf16, zero past n_rows and past D)
      if (stage_r) {
        constexpr int CPR = DP / 8;
        for (int u = tid; u < kCols * CPR; u += kThreads) {
          const int c = u / CPR;
          const int d0 = (u - c * CPR) * 8;
          const float4 z = float4{0.f, 0.f, 0.f, 0.f};
          mf_bf16x8 a = pack_bf16(z, z), bb = a;
          if (rb0 + c < n_rows) {
            const size_t row = rbase + row_list[rb0 + c];
            a = pack_bf16(ld4(t_rs, row, d0, D, p.dtype, vec), ld4(t_rs, row, d0 + 4, D, p.dtype, vec));
            bb = pack_bf16(ld4(t_rp, row, d0, D, dt_rp, vec), ld4(t_rp, row, d0 + 4, D, dt_rp, vec));
          }
          *reinterpret_cast<mf_bf16x8*>(RS16 + c * KS + d0) = a;
          *reinterpret_cast<mf_bf16x8*>(RP16 + c * KS + d0) = bb;
        }
      }
    }
    // per-wave bias sums (only this wave touches them: no barrier needed)
    if (has_bias && rbi == 0) {
      for (int u = lane; u < kCols; u += 64) wcol[wave * kCols + u] = 0.0f;
      if (cbi == 0)
        for (int u = lane; u < NP; u += 64) wrow[wave * NP + u] = 0.0f;
    }
    if (stage || stage_r) __syncthreads();
    if (!active) continue;

    // column-tile validity of this block
    const int nkt = (ncols + 15) / 16;
    uint32_t pv_outer[2] = {0xffffffffu, 0xffffffffu};
    if constexpr (ROLE != kRoleQ) {
      if (has_pv) {
        pv_outer[0] = pvb[2 * ol];
        pv_outer[1] = pvb[2 * ol + 1];
      }
    }
    const float gq_o = gate_o * kLog2e;

    const int n_rt = M16 ? (min(kCols, n_rows - rb0) + 15) / 16 : (n_rows + 15) / 16;
    for (int rt = 0; rt < n_rt; ++rt) {
      const int row = rb0 + rt * 16 + r16;  // compacted row index
      const bool row_ok = row < n_rows;
      const size_t rrow = rbase + (row_ok ? row_list[row] : 0);
      const int ro = row_ok ? row_list[row] : 0;
      float4 rs[NT], rp[NT];  // row values at d = dof(t, g) + e
      if constexpr (M16) {
        const __bf16* rsp = RS16 + (rt * 16 + r16) * KS + 8 * g;
        const __bf16* rpp = RP16 + (rt * 16 + r16) * KS + 8 * g;
#pragma unroll
        for (int s = 0; s < NT / 2; ++s) {
          const mf_bf16x8 a = *reinterpret_cast<const mf_bf16x8*>(rsp + 32 * s);
          const mf_bf16x8 bb = *reinterpret_cast<const mf_bf16x8*>(rpp + 32 * s);
          rs[2 * s] = bf16_lo(a);
          rs[2 * s + 1] = bf16_hi(a);
          rp[2 * s] = bf16_lo(bb);
          rp[2 * s + 1] = bf16_hi(bb);
        }
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          rs[t] = row_ok ? ld4(t_rs, rrow, dof<M16>(t, g), D, p.dtype, vec) : float4{0.f, 0.f, 0.f, 0.f};
          rp[t] = row_ok ? ld4(t_rp, rrow, dof<M16>(t, g), D, dt_rp, vec) : float4{0.f, 0.f, 0.f, 0.f};
        }
      }
      // per-row softmax state: the query's lse (log2) and delta
      float lse2_r = lse2_o, delta_r = delta_o, gate_r = gate_o, gq_r = gq_o;
      if constexpr (ROLE != kRoleQ) {
        lse2_r = row_ok ? lse2q[row] : 0.0f;
        delta_r = row_ok ? delta[row] : 0.0f;
        if (has_bias) {
          gate_r = row_ok ? ld1(p.gate, rrow, p.bias_dtype) : 0.0f;
          gq_r = gate_r * kLog2e;
        }
      }
      uint32_t pv_row[2] = {pv_outer[0], pv_outer[1]};
      if constexpr (ROLE == kRoleQ) {
        if (has_pv) {
          pv_row[0] = row_ok ? pvb[2 * row] : 0u;
          pv_row[1] = row_ok ? pvb[2 * row + 1] : 0u;
        }
      }
      // bias term that depends on (outer, row) only
      float bias_row = 0.0f;
      if (has_bias && row_ok) {
        if constexpr (ROLE == kRoleQ) bias_row = ld1(p.u, orow * N + ro, p.bias_dtype);   // u[i=o][j=r]
        if constexpr (ROLE == kRoleJ) bias_row = ld1(p.u, rrow * N + oo, p.bias_dtype);   // u[i=r][j=o]
        if constexpr (ROLE == kRoleK) bias_row = ld1(p.vb, rrow * N + oo, p.bias_dtype);  // v[i=r][k=o]
      }

      // GEMM1 (S^T) and GEMM1' (dP^T): lane holds row r16 and columns 16 kt + 4 g + r
      mf_f32x4 sv[4], dv[4];
      if constexpr (M16) {
        // B operands: row r16, d = 32 s + 8 g .. +7, products rounded to bf16
        constexpr int NS = DP / 32;
        mf_bf16x8 bs[NS], bp[NS], bpl[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          bs[s] = pack_bf16(mul4(rs[2 * s], oS[2 * s]), mul4(rs[2 * s + 1], oS[2 * s + 1]));
          // dP operand as bf16 hi + lo: dP - delta cancels when one pair dominates the softmax
          const float4 x0 = mul4(rp[2 * s], oP[2 * s]), x1 = mul4(rp[2 * s + 1], oP[2 * s + 1]);
          bp[s] = pack_bf16(x0, x1);
          const float4 h0 = bf16_lo(bp[s]), h1 = bf16_hi(bp[s]);
          bpl[s] = pack_bf16(float4{x0.x - h0.x, x0.y - h0.y, x0.z - h0.z, x0.w - h0.w},
                             float4{x1.x - h1.x, x1.y - h1.y, x1.z - h1.z, x1.w - h1.w});
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          sv[kt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
          dv[kt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
          if (kt < nkt) {
            const __bf16* cs = CS16 + (kt * 16 + r16) * KS + 8 * g;
            const __bf16* cp = CP16 + (kt * 16 + r16) * KS + 8 * g;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
              const mf_bf16x8 as = *reinterpret_cast<const mf_bf16x8*>(cs + 32 * s);
              const mf_bf16x8 ap = *reinterpret_cast<const mf_bf16x8*>(cp + 32 * s);
              sv[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as, bs[s], sv[kt], 0, 0, 0);
              dv[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap, bp[s], dv[kt], 0, 0, 0);
              dv[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap, bpl[s], dv[kt], 0, 0, 0);
            }
          }
        }
      } else {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        sv[kt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        dv[kt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        if (kt < nkt) {
          const float* cs = CS + (kt * 16 + r16) * D4 + 4 * g;
          const float* cp = CP + (kt * 16 + r16) * D4 + 4 * g;
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const float4 as = *reinterpret_cast<const float4*>(cs + 16 * t);
            const float4 ap = *reinterpret_cast<const float4*>(cp + 16 * t);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              sv[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4(as, e), f4(rs[t], e) * f4(oS[t], e), sv[kt], 0, 0, 0);
              dv[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4(ap, e), f4(rp[t], e) * f4(oP[t], e), dv[kt], 0, 0, 0);
            }
          }
        }
      }
      }

      // ---- low-rank terms of the lane's 16 pairs (LR): A into S, M into dP ----
      // column x of the lane: kt = x >> 2, r = x & 3, block column 16 kt + 4 g + r
      float la[16], lm[16];
      int catom[16];
      uint32_t cokm = 0u;  // bit x: column x is a valid key
      size_t qrow = 0;     // the query of the lane's pairs (row of [B*H, N])
      float agl2 = 0.0f;   // ag_i Ra^-1/2 log2(e)
      if constexpr (LR) {
        qrow = ROLE == kRoleQ ? orow : rrow;
        const int rowkey = ROLE == kRoleQ ? ro : oo;  // Q: j = row; J: j = o; K: k = o
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int c = (x >> 2) * 16 + 4 * g + (x & 3);
          cokm |= ((x >> 2) < nkt && cb0 + c < nk) ? (1u << x) : 0u;
          catom[x] = kidx[min(cb0 + c, nk - 1)];
          la[x] = 0.0f;
          lm[x] = 0.0f;
        }
        const size_t rowoff = qrow * N + rowkey;  // [.., N, N, R] row of the row-constant factor
        const size_t coloff = qrow * N;           // + the column atom
        if (p.al) {
          agl2 = p.ag[qrow] * p.a_scale * kLog2e;
          const float* rowp = (ROLE == kRoleK ? p.ar : p.al) + rowoff * p.Ra;
          const float* colp = (ROLE == kRoleK ? p.al : p.ar) + coloff * p.Ra;
          for (int c0 = 0; c0 < p.Ra; c0 += 4) {
            const float4 rv = row_ok ? ld_r4(rowp + c0, p.Ra - c0, p.lr_vec) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int x = 0; x < 16; ++x) {
              if (!((cokm >> x) & 1u)) continue;
              const float4 cv = ld_r4(colp + size_t(catom[x]) * p.Ra + c0, p.Ra - c0, p.lr_vec);
              la[x] = fmaf(rv.w, cv.w, fmaf(rv.z, cv.z, fmaf(rv.y, cv.y, fmaf(rv.x, cv.x, la[x]))));
            }
          }
        }
        if (p.ml) {
          const float* rowp = (ROLE == kRoleK ? p.mr : p.ml) + rowoff * p.Rm;
          const float* colp = (ROLE == kRoleK ? p.ml : p.mr) + coloff * p.Rm;
          const float* dcp = p.dc + qrow * p.Rm;
          for (int c0 = 0; c0 < p.Rm; c0 += 4) {
            float4 rv = float4{0.f, 0.f, 0.f, 0.f};
            if (row_ok) rv = mul4(ld_r4(rowp + c0, p.Rm - c0, p.lr_vec), ld_r4(dcp + c0, p.Rm - c0, p.lr_vec));
#pragma unroll
            for (int x = 0; x < 16; ++x) {
              if (!((cokm >> x) & 1u)) continue;
              const float4 cv = ld_r4(colp + size_t(catom[x]) * p.Rm + c0, p.Rm - c0, p.lr_vec);
              lm[x] = fmaf(rv.w, cv.w, fmaf(rv.z, cv.z, fmaf(rv.y, cv.y, fmaf(rv.x, cv.x, lm[x]))));
            }
          }
        }
      }

      // P, dS (sv <- dS, dv <- P) and the bias sums
      float rowsum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = kt * 16 + 4 * g + r;  // column within the block
          const bool col_ok = kt < nkt && cb0 + c < nk;
          const bool ok = row_ok && col_ok && ((pv_row[c >> 5] >> (c & 31)) & 1u);
          float s2 = sv[kt][r];
          float base = 0.0f;
          if (has_bias && ok) {
            const int co = kidx[cb0 + c];
            float be, bc;  // terms of (row, col) and of (outer, col)
            if constexpr (ROLE == kRoleQ) {
              bc = ld1(p.vb, orow * N + co, p.bias_dtype);            // v[i=o][k=c]
              be = ld1(p.w, (rbase + ro) * N + co, p.bias_dtype);     // w[j=r][k=c]
            } else if constexpr (ROLE == kRoleJ) {
              be = ld1(p.vb, rrow * N + co, p.bias_dtype);            // v[i=r][k=c]
              bc = ld1(p.w, orow * N + co, p.bias_dtype);             // w[j=o][k=c]
            } else {
              be = ld1(p.u, rrow * N + co, p.bias_dtype);             // u[i=r][j=c]
              bc = ld1(p.w, (rbase + co) * N + oo, p.bias_dtype);     // w[j=c][k=o]
            }
            base = (bias_row + be) + bc;
            s2 = fmaf(gq_r, base, s2);
          }
          float dpv = dv[kt][r];
          if constexpr (LR) {
            if (p.al) s2 = fmaf(agl2, la[kt * 4 + r], s2);
            if (p.ml) dpv = fmaf(p.m_scale, lm[kt * 4 + r], dpv);
          }
          const float pe = ok ? fast_exp2(s2 - lse2_r) : 0.0f;
          const float ds = pe * (dpv - delta_r);
          sv[kt][r] = ds;
          dv[kt][r] = pe;
          if constexpr (ROLE == kRoleQ) {
            rowsum += ds;
            gacc = fmaf(ds, base, gacc);
            if constexpr (LR) gacc_a = fmaf(ds, la[kt * 4 + r], gacc_a);
          }
        }
      }

      // bias sums: role Q du (row sums) and dv (column sums), role J dw (column sums of gate_r dS)
      if (has_bias) {
        if constexpr (ROLE == kRoleQ) {
          rowsum = rows4_sum(rowsum);
          if (g == 0 && row_ok) wrow[wave * NP + row] += rowsum;
        }
        if constexpr (ROLE != kRoleK) {
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float x = ROLE == kRoleQ ? sv[kt][r] : gate_r * sv[kt][r];
              x = row16_sum(x);
              if (r16 == 0) wcol[wave * kCols + kt * 16 + 4 * g + r] += x;
            }
        }
      }

      // ---- gradients of the low-rank terms (LR): role Q sums over its columns k into dangle_left[o][row],
      // dmessage_left[o][row] (and the row's sum_k P ML MR partial), role K over its columns j into
      // dangle_right[row][o], dmessage_right[row][o]; each (query, key) entry is one lane's, added per
      // column block in block order ----
      if constexpr (LR && ROLE != kRoleJ) {
        const size_t dstoff = ROLE == kRoleQ ? qrow * N + ro : qrow * N + oo;
        const size_t coloff = qrow * N;
        float* dA = ROLE == kRoleQ ? p.dal : p.dar;
        if (p.al && dA) {
          const float* colp = (ROLE == kRoleK ? p.al : p.ar) + coloff * p.Ra;
          const float gs = p.ag[qrow] * p.a_scale;
          for (int c0 = 0; c0 < p.Ra; c0 += 4) {
            float4 t = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int x = 0; x < 16; ++x) {
              if (!((cokm >> x) & 1u)) continue;
              const float4 cv = ld_r4(colp + size_t(catom[x]) * p.Ra + c0, p.Ra - c0, p.lr_vec);
              const float d = sv[x >> 2][x & 3];
              t = float4{fmaf(d, cv.x, t.x), fmaf(d, cv.y, t.y), fmaf(d, cv.z, t.z), fmaf(d, cv.w, t.w)};
            }
            t = sum_groups4(t);
            if (g == 0 && row_ok) {
              float* dst = dA + dstoff * p.Ra + c0;
              const int rem = min(4, p.Ra - c0);
              dst[0] = fmaf(gs, t.x, dst[0]);
              if (rem > 1) dst[1] = fmaf(gs, t.y, dst[1]);
              if (rem > 2) dst[2] = fmaf(gs, t.z, dst[2]);
              if (rem > 3) dst[3] = fmaf(gs, t.w, dst[3]);
            }
          }
        }
        float* dM = ROLE == kRoleQ ? p.dml : p.dmr;
        const bool want_m = dM != nullptr || (ROLE == kRoleQ && p.coeff != nullptr);
        if (p.ml && want_m) {
          const float* colp = (ROLE == kRoleK ? p.ml : p.mr) + coloff * p.Rm;
          const float* dcp = p.dc + qrow * p.Rm;
          const float* mlrow = p.ml + (qrow * N + ro) * p.Rm;  // role Q: ML[o][row]
          for (int c0 = 0; c0 < p.Rm; c0 += 4) {
            float4 t = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int x = 0; x < 16; ++x) {
              if (!((cokm >> x) & 1u)) continue;
              const float4 cv = ld_r4(colp + size_t(catom[x]) * p.Rm + c0, p.Rm - c0, p.lr_vec);
              const float pe = dv[x >> 2][x & 3];
              t = float4{fmaf(pe, cv.x, t.x), fmaf(pe, cv.y, t.y), fmaf(pe, cv.z, t.z), fmaf(pe, cv.w, t.w)};
            }
            t = sum_groups4(t);
            if (g == 0 && row_ok) {
              const int rem = min(4, p.Rm - c0);
              if (dM) {
                const float4 dcv = ld_r4(dcp + c0, rem, p.lr_vec);
                float* dst = dM + dstoff * p.Rm + c0;
                dst[0] = fmaf(p.m_scale * dcv.x, t.x, dst[0]);
                if (rem > 1) dst[1] = fmaf(p.m_scale * dcv.y, t.y, dst[1]);
                if (rem > 2) dst[2] = fmaf(p.m_scale * dcv.z, t.z, dst[2]);
                if (rem > 3) dst[3] = fmaf(p.m_scale * dcv.w, t.w, dst[3]);
              }
              if constexpr (ROLE == kRoleQ) {
                if (p.coeff) {
                  const float4 mv = ld_r4(mlrow + c0, rem, p.lr_vec);
                  float* cl = coeffL + (wave * 16 + r16) * p.RmP + c0;
                  cl[0] = fmaf(mv.x, t.x, cl[0]);
                  cl[1] = fmaf(mv.y, t.y, cl[1]);
                  cl[2] = fmaf(mv.z, t.z, cl[2]);
                  cl[3] = fmaf(mv.w, t.w, cl[3]);
                }
              }
            }
          }
        }
      }

      // GEMM2: C2a[d][r] = sum_c C_S[c][d] dS[r][c];  C2b[d][r] = sum_c C_P[c][d] P[r][c] (roles J, K)
      if constexpr (M16) {
        // K step pr covers columns 32 pr .. +31; k slot 8 g + j is column
        // 32 pr + 4 g + j (j < 4, tile 2 pr) or 32 pr + 16 + 4 g + j - 4
        // (tile 2 pr + 1): the columns this lane holds in sv / dv.  The A
        // operand rows of lane (g, r16) are d = dof(t, r16 >> 2) + (r16 & 3):
        // lane 4 e + a of group g addresses column 32 pr + 4 g + e (+16),
        // d = 32 s + 8 a + 4 h .. +3, and read_tr16 hands lane 4 a + c the
        // four columns' element c.
        mf_bf16x8 ps[2], pp[2];
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          ps[pr] = pack_bf16(float4{sv[2 * pr][0], sv[2 * pr][1], sv[2 * pr][2], sv[2 * pr][3]},
                             float4{sv[2 * pr + 1][0], sv[2 * pr + 1][1], sv[2 * pr + 1][2], sv[2 * pr + 1][3]});
          pp[pr] = pack_bf16(float4{dv[2 * pr][0], dv[2 * pr][1], dv[2 * pr][2], dv[2 * pr][3]},
                             float4{dv[2 * pr + 1][0], dv[2 * pr + 1][1], dv[2 * pr + 1][2], dv[2 * pr + 1][3]});
        }
        const int tr_off = (4 * g + (r16 >> 2)) * KS + 8 * (r16 & 3);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int toff = tr_off + 32 * (t >> 1) + 4 * (t & 1);
          mf_f32x4 ca = mf_f32x4{0.f, 0.f, 0.f, 0.f}, cb = ca;
#pragma unroll
          for (int pr = 0; pr < 2; ++pr) {
            if (2 * pr >= nkt) continue;
            const __bf16* pa = CS16 + toff + 32 * pr * KS;
            const mf_bf16x8 aa = __builtin_shufflevector(read_tr16(pa), read_tr16(pa + 16 * KS), 0, 1, 2, 3, 4, 5, 6, 7);
            ca = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa, ps[pr], ca, 0, 0, 0);
            if constexpr (ROLE != kRoleQ) {
              const __bf16* pb = CP16 + toff + 32 * pr * KS;
              const mf_bf16x8 ab =
                  __builtin_shufflevector(read_tr16(pb), read_tr16(pb + 16 * KS), 0, 1, 2, 3, 4, 5, 6, 7);
              cb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, pp[pr], cb, 0, 0, 0);
            }
          }
          // out_o[d] += R[r][d] C2[d][r]: ca[r] is d = dof(t, g) + r of row r16, as is rs[t]
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc_a[t][r] = fmaf(f4(rs[t], r), ca[r], acc_a[t][r]);
            if constexpr (ROLE != kRoleQ) acc_b[t][r] = fmaf(f4(rp[t], r), cb[r], acc_b[t][r]);
          }
        }
        continue;
      }
      mf_f32x4 c2a[NT], c2b[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        c2a[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        c2b[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        if (kt >= nkt) continue;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int c = kt * 16 + 4 * g + rr;
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            c2a[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(CS[c * D4 + 16 * t + r16], sv[kt][rr], c2a[t], 0, 0, 0);
            if constexpr (ROLE != kRoleQ)
              c2b[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(CP[c * D4 + 16 * t + r16], dv[kt][rr], c2b[t], 0, 0, 0);
          }
        }
      }
      // out_o[d] += R[r][d] C2[d][r]: lane holds d = 16 t + 4 g + r of row r16, which is rs[t] / rp[t]
      if (row_ok) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc_a[t][r] = fmaf(f4(rs[t], r), c2a[t][r], acc_a[t][r]);
            if constexpr (ROLE != kRoleQ) acc_b[t][r] = fmaf(f4(rp[t], r), c2b[t][r], acc_b[t][r]);
          }
      }
    }

  }  // rbi
    // column sums of this block are complete: dv_bias (role Q) and dw (role J)
    if constexpr (ROLE != kRoleK) {
      if (has_bias && active) {
        for (int c = lane; c < ncols; c += 64) {
          const size_t dst = orow * N + kidx[cb0 + c];
          if constexpr (ROLE == kRoleQ) {
            if (p.dvb) store_grad(p.dvb, dst, gate_o * wcol[wave * kCols + c], p.gout16);
          } else {
            if (p.dw) store_grad(p.dw, dst, wcol[wave * kCols + c], p.gout16);
          }
        }
      }
    }
  }
  if (!active) continue;  // uniform over the wave

  // ---- write the outer index's rows: sum over the 16 row lanes of each group ----
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc_a[t][r] = group16_sum(acc_a[t][r]);
      if constexpr (ROLE != kRoleQ) acc_b[t][r] = group16_sum(acc_b[t][r]);
    }
  void* out_a = ROLE == kRoleQ ? p.dq : (ROLE == kRoleJ ? p.dk1 : p.dk2);
  void* out_b = ROLE == kRoleQ ? nullptr : (ROLE == kRoleJ ? p.dv1 : p.dv2);
  // lane (g, r16) writes d = dof(t, g) + (r16 & 3) for the tiles t with (t & 3) == r16 >> 2
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if ((t & 3) != (r16 >> 2)) continue;
    const int d = dof<M16>(t, g) + (r16 & 3);
    if (d >= D) continue;
    float va = 0.0f, vb = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if ((r16 & 3) == r) {
        va = acc_a[t][r];
        vb = acc_b[t][r];
      }
    if (out_a) store_grad(out_a, orow * D + d, va, p.gout16);
    if (out_b) store_grad(out_b, orow * D + d, vb, p.gout16);
  }
  if constexpr (LR && ROLE == kRoleQ) {
    if (p.al && p.dag) {
      const float dg = wave_sum(gacc_a);
      if (lane == 0) p.dag[orow] = p.a_scale * dg;
    }
    if (p.ml && p.coeff) {
      __builtin_amdgcn_wave_barrier();  // the row lanes' partials (LDS, this wave's own) are written
      for (int r = lane; r < p.Rm; r += 64) {
        float c = 0.0f;
        for (int x = 0; x < 16; ++x) c += coeffL[(wave * 16 + x) * p.RmP + r];
        p.coeff[orow * p.Rm + r] = c;
      }
    }
  }
  if constexpr (ROLE == kRoleQ) {
    if (has_bias) {
      const float dg = wave_sum(gacc);
      if (lane == 0 && p.dgate) store_grad(p.dgate, orow, dg, p.gout16);
      if (p.du)
        for (int row = lane; row < nk; row += 64)
          store_grad(p.du, orow * N + kidx[row], gate_o * wrow[wave * NP + row], p.gout16);
    }
  }
  }  // it
}

// One kernel per role: each gets its own register allocation.
// All three roles in one launch: blocks [r G, (r + 1) G) run role r (G =
// B H OB).  The roles write disjoint gradients, so they may run
// concurrently, and one launch lets the uneven blocks of the three roles
// (work grows with the cube of a molecule's size) fill each other's tails.
template <int DP, bool M16, bool BIAS, bool LR>
__global__ void __launch_bounds__((Shape<DP, M16, LR>::kThreads), (Shape<DP, M16, LR>::kMinBlocks)) simplicial_bwd_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  if (p.served != nullptr && *p.unserved == 0) return;  // the pair kernel served every molecule
  const int G = p.B * p.H * p.OB;
  const int* served = reinterpret_cast<const int*>(smem + p.served_lds);
  if (p.served != nullptr) {
    for (int i = threadIdx.x; i < p.B; i += Shape<DP, M16, LR>::kThreads)
      const_cast<int*>(served)[i] = p.served[i];
    __syncthreads();
  }
  for (int w = blockIdx.x; w < p.blocks; w += gridDim.x) {
    const int role = w / G;
    const int blk = w - role * G;
    const int bh = blk / p.OB;
    const int ob = blk - bh * p.OB;
    if (p.served != nullptr && served[bh / p.H] != 0) continue;  // uniform: the pair kernel's molecule
    if (w != int(blockIdx.x)) __syncthreads();  // the previous block's LDS reads are done
    if (role == kRoleQ) run_role<DP, kRoleQ, M16, BIAS, LR>(p, smem, bh, ob);
    else if (role == kRoleJ) run_role<DP, kRoleJ, M16, BIAS, LR>(p, smem, bh, ob);
    else run_role<DP, kRoleK, M16, BIAS, LR>(p, smem, bh, ob);
  }
}

// dc[row][r] = basis[h][r] . go[row] for every row of [B*H, N] (message term), and coeff[row][r] = 0:
// one thread per (row, r).
__global__ void __launch_bounds__(256) lr_dc_kernel(Params p) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = (long long)p.B * p.H * p.N * p.Rm;
  if (idx >= total) return;
  const int r = int(idx % p.Rm);
  const long long row = idx / p.Rm;
  const int h = int((row / p.N) % p.H);
  const float* bs = p.mb + (size_t(h) * p.Rm + r) * p.D;
  float acc = 0.0f;
  for (int d = 0; d < p.D; ++d) acc = fmaf(bs[d], ld1(p.go, size_t(row) * p.D + d, p.gdtype), acc);
  p.dc[idx] = acc;
  // the per-query coefficients start at 0: queries of a molecule without valid keys get no role-Q wave
  if (p.coeff) p.coeff[idx] = 0.0f;
}

// dbasis[h][r][d] = Rm^-1/2 sum over valid (b, i) of coeff[b,h,i][r] go[b,h,i][d]: one workgroup per (h, r);
// thread t takes d = t % 64 (+ 64 per pass) and every fourth (b, i); the four partial sums meet in a fixed order.
__global__ void __launch_bounds__(256) lr_dbasis_kernel(Params p, float* dmb) {
  __shared__ float part[256];
  const int h = blockIdx.x, r = blockIdx.y;
  const int t = threadIdx.x;
  const int dl = t & 63, q4 = t >> 6;
  const int BN = p.B * p.N;
  for (int d0 = 0; d0 < p.D; d0 += 64) {
    const int d = d0 + dl;
    float acc = 0.0f;
    if (d < p.D) {
      for (int u = q4; u < BN; u += 4) {
        const int b = u / p.N, i = u - b * p.N;
        if (!p.qv[u]) continue;
        const size_t row = (size_t(b) * p.H + h) * p.N + i;
        acc = fmaf(p.coeff[row * p.Rm + r], ld1(p.go, row * p.D + d, p.gdtype), acc);
      }
    }
    part[t] = acc;
    __syncthreads();
    if (q4 == 0 && d < p.D)
      dmb[(size_t(h) * p.Rm + r) * p.D + d] = p.m_scale * (((part[dl] + part[64 + dl]) + part[128 + dl]) + part[192 + dl]);
    __syncthreads();
  }
}

// 16-bit gradients are written in full: zeros at every row the kernels do not write -- padded queries (dq) and
// keys (dk1, dv1, dk2, dv2), and every row of a molecule without a valid query or key.  One workgroup per
// (molecule, head): the two mask rows are read once into LDS, then 16-byte stores of zeros.
constexpr int kZeroMaxN = 4096;
__global__ void __launch_bounds__(256) zero_rows_kernel(Params p) {
  __shared__ uint8_t s_q[kZeroMaxN], s_k[kZeroMaxN];
  __shared__ int s_cnt[2];
  const int bh = blockIdx.x;
  const int b = bh / p.H;
  const int N = p.N, D = p.D;
  const int tid = threadIdx.x;
  if (tid < 2) s_cnt[tid] = 0;
  __syncthreads();
  int cq = 0, ck = 0;
  for (int t = tid; t < N; t += 256) {
    const uint8_t q = p.qv[size_t(b) * N + t] != 0, k = p.pkv[size_t(b) * N + t] != 0;
    s_q[t] = q;
    s_k[t] = k;
    cq += q;
    ck += k;
  }
  if (cq) atomicAdd(&s_cnt[0], cq);
  if (ck) atomicAdd(&s_cnt[1], ck);
  __syncthreads();
  const bool empty = s_cnt[0] == 0 || s_cnt[1] == 0;
  const int C = D / 8;  // 16-byte chunks per row (D % 8 == 0 on this path)
  const size_t base = size_t(bh) * N * C;
  const uint4 z{0u, 0u, 0u, 0u};
  for (int u = tid; u < N * C; u += 256) {
    const int row = u / C;
    if (empty || !s_q[row]) static_cast<uint4*>(p.dq)[base + u] = z;
    if (empty || !s_k[row]) {
      static_cast<uint4*>(p.dk1)[base + u] = z;
      static_cast<uint4*>(p.dv1)[base + u] = z;
      static_cast<uint4*>(p.dk2)[base + u] = z;
      static_cast<uint4*>(p.dv2)[base + u] = z;
    }
  }
}

// bf16 bias gradients are written in full: the four tensors are cleared first (one flat pass of 16-byte
// stores, the last n % 8 elements one by one), then the kernels write every valid entry.
__global__ void __launch_bounds__(256) zero_bias_kernel(void* du, void* dvb, void* dw, void* dgate, size_t plane,
                                                        size_t gates) {
  void* const ptrs[4] = {du, dvb, dw, dgate};
  const size_t n[4] = {plane, plane, plane, gates};
  const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (ptrs[t] == nullptr) continue;
    const size_t chunks = n[t] / 8;
    for (size_t c = gid; c < chunks; c += stride) static_cast<uint4*>(ptrs[t])[c] = uint4{0u, 0u, 0u, 0u};
    if (gid < n[t] % 8) static_cast<__bf16*>(ptrs[t])[chunks * 8 + gid] = __bf16(0.0f);
  }
}

template <int DP, bool M16, bool LR = false>
int launch(Params prm, bool has_pv, bool has_bias, hipStream_t stream) {
  size_t lds = Lay<DP, M16, LR>::bytes(prm.NP, has_pv, has_bias, (LR && prm.ml && prm.coeff) ? prm.RmP : 0);
  lds = (lds + 15) & ~size_t(15);
  prm.served_lds = int(lds);
  if (prm.served != nullptr) lds += size_t(prm.B) * 4;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  if (lds > size_t(dev.max_lds_per_block))
    return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_bwd: tokens=" + std::to_string(prm.N) + " needs " +
                                        std::to_string(lds) + " bytes of LDS per workgroup, the device offers " +
                                        std::to_string(dev.max_lds_per_block));
  using Kern = void (*)(Params);
  const Kern kerns[2] = {simplicial_bwd_kernel<DP, M16, false, LR>, simplicial_bwd_kernel<DP, M16, true, LR>};
  st = ensure_dynamic_lds(reinterpret_cast<const void*>(kerns[has_bias]), 160 * 1024);
  if (st != MF_OK) return st;
  // about 8 workgroups per CU for each role, at most one per kWaves outer indices
  const long long bh = (long long)prm.B * prm.H;
  const long long want = (8LL * dev.num_cus + bh - 1) / bh;
  constexpr int kW = Shape<DP, M16, LR>::kWaves;
  prm.OB = int(std::max(1LL, std::min<long long>(want, (prm.N + kW - 1) / kW)));
  const long long blocks = 3 * bh * prm.OB;
  if (blocks > 0x7fffffffLL) return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_bwd: grid too large");
  prm.blocks = int(blocks);
  // after the pair kernel most blocks are skipped: a grid of a few workgroups per CU loops over them
  const long long grid = prm.served != nullptr ? std::min<long long>(blocks, 2LL * dev.num_cus) : blocks;
  hipLaunchKernelGGL(kerns[has_bias], dim3(unsigned(grid)), dim3(Shape<DP, M16, LR>::kThreads), lds, stream, prm);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

}  // namespace sbwd
}  // namespace mf

using namespace mf;

// dc and the per-query coefficients of the message term, [B*H, N, Rm] fp32 each
static uint64_t message_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens, int32_t message_rank) {
  if (batch <= 0 || heads <= 0 || tokens <= 0 || message_rank <= 0) return 0;
  return 2ull * uint64_t(batch) * uint64_t(heads) * uint64_t(tokens) * uint64_t(message_rank) * 4ull;
}

extern "C" int mf_simplicial_bwd(const mf_simplicial_bwd_args* a, void* stream) {
  using namespace mf::sbwd;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: args is NULL");
  if (!a->q || !a->k1 || !a->v1 || !a->k2 || !a->v2 || !a->grad_out || !a->out || !a->lse)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: q, k1, v1, k2, v2, grad_out, out and lse must be non-NULL");
  if (!a->query_valid || !a->pair_key_valid)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: query_valid and pair_key_valid must be non-NULL");
  if (a->batch <= 0 || a->heads <= 0 || a->tokens <= 0 || a->head_dim <= 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: batch, heads, tokens and head_dim must be positive");
  if (a->head_dim > 128)
    return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_bwd only supports head_dim <= 128, got " + std::to_string(a->head_dim));
  for (int dt : {a->dtype, a->grad_dtype})
    if (dt != MF_DTYPE_F32 && dt != MF_DTYPE_F16 && dt != MF_DTYPE_BF16)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: unknown dtype " + std::to_string(dt));
  const bool has_bias = a->bias_u != nullptr;
  if (has_bias) {
    if (!a->bias_v || !a->bias_w || !a->bias_gate)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: bias_u, bias_v, bias_w and bias_gate go together");
    if (a->bias_dtype != MF_DTYPE_F32 && a->bias_dtype != MF_DTYPE_F16 && a->bias_dtype != MF_DTYPE_BF16)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: unknown bias_dtype " + std::to_string(a->bias_dtype));
  } else if (a->du || a->dv_bias || a->dw || a->dgate) {
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: bias gradients requested without a bias");
  }
  const bool has_angle = a->angle_left != nullptr;
  const bool has_msg = a->message_left != nullptr;
  if (has_angle) {
    if (!a->angle_right || !a->angle_gate)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: angle_left, angle_right and angle_gate go together");
    if (a->angle_rank < 1 || a->angle_rank > 64)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: angle_rank must be in 1..64, got " + std::to_string(a->angle_rank));
  } else if (a->dangle_left || a->dangle_right || a->dangle_gate) {
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: angle gradients requested without an angle term");
  }
  if (has_msg) {
    if (!a->message_right || !a->message_basis)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: message_left, message_right and message_basis go together");
    if (a->message_rank < 1 || a->message_rank > 64)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: message_rank must be in 1..64, got " + std::to_string(a->message_rank));
    const uint64_t need = message_workspace_bytes(a->batch, a->heads, a->tokens, a->message_rank);
    if (a->workspace == nullptr || a->workspace_bytes < need)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: the message term needs " + std::to_string(need) +
                                               " bytes of workspace (mf_simplicial_bwd_workspace_size)");
    if (reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: workspace must be 16-byte aligned");
  } else if (a->dmessage_left || a->dmessage_right || a->dmessage_basis) {
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: message gradients requested without a message term");
  }
  const bool gout16 = a->grads_dtype == MF_DTYPE_BF16;
  if (a->grads_dtype != MF_DTYPE_F32 && !gout16)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: grads_dtype must be MF_DTYPE_F32 or MF_DTYPE_BF16");
  if (gout16) {
    if (a->dtype != MF_DTYPE_BF16 || a->grad_dtype != MF_DTYPE_BF16 || has_angle || has_msg)
      return fail(MF_ERR_INVALID_ARGUMENT,
                  "mf_simplicial_bwd: bf16 gradients need bf16 operands and grad_out and no low-rank term");
    if (!a->dq || !a->dk1 || !a->dv1 || !a->dk2 || !a->dv2 || a->head_dim % 8 != 0 || a->tokens > kZeroMaxN)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: bf16 gradients need all five of dq, dk1, dv1, dk2, "
                                           "dv2, a head_dim that is a multiple of 8 and at most 4096 tokens");
    for (const void* ptr : {a->dq, a->dk1, a->dv1, a->dk2, a->dv2, a->du, a->dv_bias, a->dw, a->dgate})
      if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0)
        return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_bwd: bf16 gradient buffers must be 16-byte aligned");
  }
  Params prm{};
  prm.gout16 = gout16 ? 1 : 0;
  prm.q = a->q; prm.k1 = a->k1; prm.v1 = a->v1; prm.k2 = a->k2; prm.v2 = a->v2; prm.go = a->grad_out;
  prm.out = a->out; prm.lse = a->lse;
  prm.qv = a->query_valid; prm.pkv = a->pair_key_valid; prm.pv = a->pair_valid;
  if (has_bias) {
    prm.u = a->bias_u; prm.vb = a->bias_v; prm.w = a->bias_w; prm.gate = a->bias_gate;
    prm.bias_dtype = a->bias_dtype;
  }
  prm.dq = a->dq; prm.dk1 = a->dk1; prm.dv1 = a->dv1; prm.dk2 = a->dk2; prm.dv2 = a->dv2;
  prm.du = a->du; prm.dvb = a->dv_bias; prm.dw = a->dw; prm.dgate = a->dgate;
  prm.B = a->batch; prm.H = a->heads; prm.N = a->tokens; prm.D = a->head_dim;
  prm.dtype = a->dtype; prm.gdtype = a->grad_dtype;
  prm.NP = (a->tokens + 63) / 64 * 64;
  // 4-element row loads need D % 4 == 0 and bases aligned to 4 elements
  bool vec = a->head_dim % 4 == 0;
  const size_t esz = a->dtype == MF_DTYPE_F32 ? 16 : 8;
  for (const void* ptr : {a->q, a->k1, a->v1, a->k2, a->v2})
    vec = vec && reinterpret_cast<uintptr_t>(ptr) % esz == 0;
  vec = vec && reinterpret_cast<uintptr_t>(a->grad_out) % (a->grad_dtype == MF_DTYPE_F32 ? 16 : 8) == 0;
  vec = vec && reinterpret_cast<uintptr_t>(a->out) % 16 == 0;
  prm.vec = vec ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool has_pv = a->pair_valid != nullptr;
  const int D = a->head_dim;
  if (has_angle || has_msg) {
    // the rank terms: fp32 arithmetic (the fp32 path) for every operand dtype, 4 waves per workgroup
    bool lv = true;
    if (has_angle) {
      prm.al = a->angle_left; prm.ar = a->angle_right; prm.ag = a->angle_gate;
      prm.Ra = a->angle_rank;
      prm.a_scale = 1.0f / std::sqrt(float(a->angle_rank));
      prm.dal = a->dangle_left; prm.dar = a->dangle_right; prm.dag = a->dangle_gate;
      lv = lv && a->angle_rank % 4 == 0;
      for (const void* ptr : {(const void*)a->angle_left, (const void*)a->angle_right})
        lv = lv && reinterpret_cast<uintptr_t>(ptr) % 16 == 0;
    }
    if (has_msg) {
      prm.ml = a->message_left; prm.mr = a->message_right; prm.mb = a->message_basis;
      prm.Rm = a->message_rank;
      prm.RmP = (a->message_rank + 3) / 4 * 4;
      prm.m_scale = 1.0f / std::sqrt(float(a->message_rank));
      prm.dml = a->dmessage_left; prm.dmr = a->dmessage_right;
      prm.dc = static_cast<float*>(a->workspace);
      prm.coeff = a->dmessage_basis ? prm.dc + size_t(a->batch) * a->heads * a->tokens * a->message_rank : nullptr;
      lv = lv && a->message_rank % 4 == 0;
      for (const void* ptr : {(const void*)a->message_left, (const void*)a->message_right})
        lv = lv && reinterpret_cast<uintptr_t>(ptr) % 16 == 0;
      const long long total = (long long)a->batch * a->heads * a->tokens * a->message_rank;
      hipLaunchKernelGGL(lr_dc_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, prm);
      MF_HIP_CHECK(hipGetLastError());
    }
    prm.lr_vec = lv ? 1 : 0;
    int st;
    if (D <= 32) st = launch<32, false, true>(prm, has_pv, has_bias, s);
    else if (D <= 64) st = launch<64, false, true>(prm, has_pv, has_bias, s);
    else st = launch<128, false, true>(prm, has_pv, has_bias, s);
    if (st != MF_OK) return st;
    if (has_msg && a->dmessage_basis) {
      hipLaunchKernelGGL(lr_dbasis_kernel, dim3(unsigned(a->heads), unsigned(a->message_rank)), dim3(256), 0, s, prm,
                         a->dmessage_basis);
      MF_HIP_CHECK(hipGetLastError());
    }
    return MF_OK;
  }
  // bf16 operands and a bf16 grad_out: bf16 MFMA (K steps of 32 d), which stages grad_out rows as bf16 (exact
  // only for a bf16 grad_out).  Everything else -- fp16 operands, or a grad_out of another dtype -- takes the
  // fp32 path, which reads every operand in its own dtype.
  if (gout16) {
    hipLaunchKernelGGL(zero_rows_kernel, dim3(unsigned(a->batch * a->heads)), dim3(256), 0, s, prm);
    MF_HIP_CHECK(hipGetLastError());
    if (has_bias && (a->du || a->dv_bias || a->dw || a->dgate)) {
      const size_t gates = size_t(a->batch) * a->heads * a->tokens, plane = gates * a->tokens;
      const size_t grid = std::min<size_t>((plane / 8 + 255) / 256, 4096);
      hipLaunchKernelGGL(zero_bias_kernel, dim3(unsigned(std::max<size_t>(grid, 1))), dim3(256), 0, s, a->du,
                         a->dv_bias, a->dw, a->dgate, plane, gates);
      MF_HIP_CHECK(hipGetLastError());
    }
  }
  if (a->dtype == MF_DTYPE_BF16 && a->grad_dtype == MF_DTYPE_BF16) {
    // molecules of at most 80 valid atoms take the pair formulation; the ownership kernel below takes the rest
    if (simplicial_pair_bwd_serves(a)) {
      const int st = simplicial_pair_bwd_launch(a, s);
      if (st != MF_OK) return st;
      if (a->tokens <= simplicial_pair_bwd_max_tokens()) return MF_OK;
      prm.served = simplicial_pair_bwd_served(a);
      prm.unserved = simplicial_pair_bwd_unserved_count(a);
    }
    if (D <= 32) return launch<32, true>(prm, has_pv, has_bias, s);
    if (D <= 64) return launch<64, true>(prm, has_pv, has_bias, s);
    return launch<128, true>(prm, has_pv, has_bias, s);
  }
  if (D <= 16) return launch<16, false>(prm, has_pv, has_bias, s);
  if (D <= 32) return launch<32, false>(prm, has_pv, has_bias, s);
  if (D <= 64) return launch<64, false>(prm, has_pv, has_bias, s);
  return launch<128, false>(prm, has_pv, has_bias, s);
}

extern "C" uint64_t mf_simplicial_bwd_workspace_size(int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                                     int32_t message_rank) {
  if (batch <= 0 || heads <= 0 || tokens <= 0) return 0;
  // the message term's coefficients, or (head_dim 64) the pair kernel's plan and partial sums; one call uses
  // at most one of them
  const uint64_t msg = message_rank > 0 ? message_workspace_bytes(batch, heads, tokens, message_rank) : 0;
  const uint64_t pair = head_dim == 64 ? uint64_t(simplicial_pair_bwd_workspace_bytes(batch, heads)) : 0;
  return std::max(msg, pair);
}

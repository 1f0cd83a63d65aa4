// 2-simplicial attention forward for gfx950 (CDNA4).
//
// Math (simplicial_attention.py:161-180,304-344; triton_simplicial_attention.py:115-329):
//   S_i[j,k] = sum_d q_i[d] k1_j[d] k2_k[d]
//   P_i      = softmax over valid (j,k) of S_i
//   out_i[d] = sum_{j,k} P_i[j,k] v1_j[d] v2_k[d]
//
// Design:
//  * Ragged packing.  Keys (the j and k atoms) are compacted per molecule from
//    pair_key_valid, and only valid queries are visited, so the work is
//    n_q * n_k^2 per (molecule, head) instead of the padded N^3.
//  * Persistent workgroups walk a balanced list of work items
//    (molecule, head, query range).  The list is derived from the masks by
//    every workgroup itself (a ballot-count over the masks), so there is no
//    host synchronisation and a single launch.
//  * Per item, the compacted K1 and K2 rows and V2^T are staged in LDS; V1 is
//    only read once per (query, j tile) in the epilogue and comes from L1/L2.
//  * Per query i and tile of 16 j-rows, two MFMA chains:
//      GEMM1  C1[k][j]   = sum_d K2[k][d] * (q_i (.) K1[j])[d]    -> S^T tile
//      GEMM2  C2[d][j]  += sum_k V2^T[d][k] * P[j][k]             -> (P V2)^T
//    The accumulator layout of GEMM1 (lane = j row, 4 consecutive keys per
//    lane group) is exactly the B-operand layout GEMM2 needs, with the K index
//    of GEMM2 permuted consistently on both operands, so P never leaves the
//    registers.  Then out_i[d] += sum_j V1[j][d] * C2[d][j] in fp32.
//  * Online softmax in the log2 domain (log2 e folded into q) with one running
//    maximum per query, rescaled lazily: only when a tile exceeds the running
//    maximum by more than kRescaleSlack, so exp2 arguments stay <= slack.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "mf_common.h"

namespace mf {
namespace simplicial {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr float kRescaleSlack = 8.0f;  // log2 units: P <= 256 between rescales
constexpr int kMaxRank = 64;           // low-rank angle / message terms
constexpr int kRankTiles = kMaxRank / 16;
constexpr int kRankSteps = kMaxRank / 4;

// Optional logit / message terms (any pointer group may be absent).
// Row indices: tensors indexed [.., i, j] use (bh*N + i)*N + j.
struct Extras {
  const void* u;     // [BH, N, N] factorized bias, element type bias_dtype
  const void* v;
  const void* w;
  const void* gate;  // [BH, N]
  int bias_dtype;
  const float* al;   // [BH, N, N, Ra] angle left / right, [BH, N] gate
  const float* ar;
  const float* ag;
  int a_rank;
  float a_scale;     // Ra^-1/2
  const float* ml;   // [BH, N, N, Rm] message left / right, [H, Rm, D] basis
  const float* mr;
  const float* mb;
  int m_rank;
  float m_scale;     // Rm^-1/2
};

__device__ __forceinline__ float load_any(const void* p, size_t idx, int dtype) {
  if (dtype == MF_DTYPE_F32) return static_cast<const float*>(p)[idx];
  if (dtype == MF_DTYPE_BF16) return static_cast<float>(static_cast<const __bf16*>(p)[idx]);
  return static_cast<float>(static_cast<const _Float16*>(p)[idx]);
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
  int B, H, N, D;
  int NP;           // LDS row capacity: N rounded up to 32
  int work_target;  // target query * key^2 units per work item
  int vec_ok;       // rows are 16-byte aligned and D*sizeof(T) % 16 == 0
  int min_keys;     // only molecules with more keys than this are processed
  int zero_rows;    // write the zero rows of invalid queries
  Extras x;         // used by the EXT instantiations only
};

// LDS geometry shared by host (sizing) and device (carving).
template <typename T, int DP>
struct Layout {
  static constexpr int kPadK = 16 / Elem<T>::kSize;  // 16 bytes of row padding
  static constexpr int KS = DP + kPadK;              // row stride of K1s/K2s
  __host__ __device__ static int vs(int NP) { return NP + kPadK; }  // row stride of V2Ts
  __host__ __device__ static size_t bytes(int NP, int B, bool has_pv) {
    size_t s = 0;
    s += size_t(2) * NP * KS * Elem<T>::kSize;  // K1s, K2s
    s += size_t(DP) * vs(NP) * Elem<T>::kSize;  // V2Ts
    s += size_t(NP) * 4 * 2;                    // kidx, qidx
    if (has_pv) s += size_t(NP) * (NP / 32) * 4;  // pair-valid bit rows
    s += size_t(B + 1) * 4 + size_t(B) * 4;     // item_off, nkq
    return (s + 15) & ~size_t(15);
  }
};

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Queries per work item for a molecule with nk keys; a multiple of kWaves
// once it reaches kWaves so every wave gets the same number of queries.
__device__ __forceinline__ int queries_per_item(int nk, int work_target) {
  const int nk2 = max(nk * nk, 1);
  int qpi = max(1, work_target / nk2);
  if (qpi >= kWaves) qpi -= qpi % kWaves;
  return qpi;
}

// Copy `count` elements of a global row (elements [e0, e0+count) of a row of
// length D) into `dst`, zero-filling past D.  count*sizeof(T) == 16.
template <typename T>
__device__ __forceinline__ void load_row_chunk16(T* dst, const T* row, int e0, int D, bool vec_ok) {
  constexpr int C = 16 / sizeof(T);
  if (vec_ok && e0 + C <= D) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(row + e0);
  } else {
#pragma unroll
    for (int e = 0; e < C; ++e) dst[e] = (e0 + e < D) ? row[e0 + e] : T(0.0f);
  }
}

// EXT instantiations add the optional terms of Params::x:
//  * factorized bias and low-rank angle are added to each S^T tile right
//    after GEMM1 (u per lane row, v and w per key; the angle tile is its own
//    fp32 MFMA chain C[k][j] = sum_r AR[k][r] AL[j][r], the layout of S^T);
//  * the message term runs a third MFMA chain beside GEMM2,
//    CM[r][j] += sum_k MR^T[r][k] P[j][k], folded as c_r += ML[j][r] CM[r][j]
//    like the value path, rescaled with it, and added as c @ basis at the end.
// All of them read their tensors from global memory (L2): they are per query
// (u, v, the rank factors) or per (b, h) (w), not shared across work items.
// EXT: 0 = no optional terms, 1 = bias / angle, 2 = bias / angle / message.
// The message term holds a rank-tile accumulator per lane beside the value
// path; EXT == 2 runs 4 waves per workgroup so that each wave may use the
// whole register file (architectural + accumulation registers).
template <int EXT>
struct Waves {
  static constexpr int kCount = EXT == 2 ? 4 : kWaves;
  static constexpr int kThreadCount = kCount * 64;
};

template <typename T, int DP, int EXT>
__global__ void __launch_bounds__(Waves<EXT>::kThreadCount) simplicial_fwd_kernel(Params p) {
  using E = Elem<T>;
  constexpr int kWaves = Waves<EXT>::kCount;
  constexpr int kThreads = Waves<EXT>::kThreadCount;
  using L = Layout<T, DP>;
  constexpr int KS = L::KS;
  constexpr int NMT = DP / 16;            // 16-wide d tiles of GEMM2 / outputs
  constexpr int KPL = E::kKPerLane;       // K elements per lane per MFMA
  constexpr int NCH = DP / E::kKPerMfma;  // MFMAs along d for GEMM1
  constexpr int C16 = 16 / sizeof(T);     // elements per 16-byte chunk

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int NP = p.NP;
  const int VS = L::vs(NP);
  const int B = p.B, H = p.H, N = p.N, D = p.D;
  const bool has_pv = p.pv != nullptr;
  const int PW = NP / 32;  // pair-valid words per row

  T* K1s = reinterpret_cast<T*>(smem);
  T* K2s = K1s + NP * KS;
  T* V2Ts = K2s + NP * KS;
  int* kidx = reinterpret_cast<int*>(V2Ts + DP * VS);
  int* qidx = kidx + NP;
  uint32_t* pvb = reinterpret_cast<uint32_t*>(qidx + NP);
  int* item_off = reinterpret_cast<int*>(pvb + (has_pv ? NP * PW : 0));
  int* nkq = item_off + (B + 1);

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;
  const int r16 = lane & 15;

  // ---- 1. per-molecule key / query counts ----
  for (int b = wave; b < B; b += kWaves) {
    int ck = 0, cq = 0;
    for (int base = 0; base < N; base += 64) {
      const int t = base + lane;
      const bool vk = t < N && p.pkv[size_t(b) * N + t] != 0;
      const bool vq = t < N && p.qv[size_t(b) * N + t] != 0;
      ck += __popcll(__ballot(vk));
      cq += __popcll(__ballot(vq));
    }
    if (lane == 0) nkq[b] = (ck << 16) | cq;
  }
  __syncthreads();

  // ---- 2. work-item offsets (exclusive scan over molecules) ----
  if (wave == 0) {
    int running = 0;
    for (int base = 0; base < B; base += 64) {
      const int b = base + lane;
      int cnt = 0;
      if (b < B) {
        const int v = nkq[b];
        const int nk = v >> 16, nq = v & 0xffff;
        if (nq > 0 && nk > p.min_keys) cnt = H * ceil_div(nq, queries_per_item(nk, p.work_target));
      }
      int x = cnt;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
      }
      if (b < B) item_off[b] = running + x - cnt;
      running += __shfl(x, 63, 64);
    }
    if (lane == 0) item_off[B] = running;
  }

  // ---- 3. zero rows of invalid queries (grid-stride) ----
  if (p.zero_rows) {
    const int CPR = ceil_div(D, 4);  // 4-element chunks per row
    const long long rows = (long long)B * H * N;
    const long long total = rows * CPR;
    for (long long idx = (long long)blockIdx.x * kThreads + tid; idx < total;
         idx += (long long)gridDim.x * kThreads) {
      const long long row = idx / CPR;
      const int ch = int(idx - row * CPR);
      const int i = int(row % N);
      const int b = int(row / ((long long)H * N));
      if (p.qv[size_t(b) * N + i] != 0) continue;
      const int d0 = ch * 4;
      for (int e = 0; e < 4 && d0 + e < D; ++e) {
        const size_t o = size_t(row) * D + d0 + e;
        if (p.out) static_cast<T*>(p.out)[o] = T(0.0f);
        if (p.out_f32) p.out_f32[o] = 0.0f;
      }
      if (ch == 0 && p.lse) p.lse[row] = 0.0f;
    }
  }
  __syncthreads();

  const int total_items = item_off[B];

  // ---- 4. work items ----
  for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (item_off[mid] <= item) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int nk = nkq[b] >> 16;
    const int nq = nkq[b] & 0xffff;
    const int qpi = queries_per_item(nk, p.work_target);
    const int splits = ceil_div(nq, qpi);
    const int local = item - item_off[b];
    const int h = local / splits;
    const int s = local - h * splits;
    const int q0 = s * qpi;
    const int q1 = min(nq, q0 + qpi);
    const int bh = b * H + h;

    // compacted key list (wave 0) and query list (wave 1)
    if (wave < 2) {
      const uint8_t* m = (wave == 0 ? p.pkv : p.qv) + size_t(b) * N;
      int* dst = wave == 0 ? kidx : qidx;
      int count = 0;
      for (int base = 0; base < N; base += 64) {
        const int t = base + lane;
        const bool v = t < N && m[t] != 0;
        const unsigned long long bal = __ballot(v);
        const int pos = count + __popcll(bal & ((1ull << lane) - 1ull));
        if (v) dst[pos] = t;
        count += __popcll(bal);
      }
    }
    __syncthreads();

    // stage K1, K2, V1 rows (row-major) and V2^T; zero-fill rows >= nk
    const int nrow = min(NP, ceil_div(nk, 32) * 32);
    {
      const T* gk1 = static_cast<const T*>(p.k1) + size_t(bh) * N * D;
      const T* gk2 = static_cast<const T*>(p.k2) + size_t(bh) * N * D;
      const T* gv2 = static_cast<const T*>(p.v2) + size_t(bh) * N * D;
      constexpr int CPR = DP / C16;  // 16-byte chunks per padded row
      const int units = nrow * CPR;
      for (int u = tid; u < units; u += kThreads) {
        const int r = u / CPR;
        const int c = u - r * CPR;
        const int e0 = c * C16;
        T* d1 = K1s + r * KS + e0;
        T* d2 = K2s + r * KS + e0;
        T tmp[C16];
        if (r < nk) {
          const size_t src = size_t(kidx[r]) * D;
          load_row_chunk16<T>(d1, gk1 + src, e0, D, p.vec_ok);
          load_row_chunk16<T>(d2, gk2 + src, e0, D, p.vec_ok);
          load_row_chunk16<T>(tmp, gv2 + src, e0, D, p.vec_ok);
        } else {
#pragma unroll
          for (int e = 0; e < C16; ++e) { d1[e] = T(0.0f); d2[e] = T(0.0f); tmp[e] = T(0.0f); }
        }
#pragma unroll
        for (int e = 0; e < C16; ++e) V2Ts[(e0 + e) * VS + r] = tmp[e];
      }
      if (has_pv) {
        const uint8_t* gpv = p.pv + size_t(b) * N * N;
        const int wpr = nrow / 32;
        for (int u = tid; u < nrow * wpr; u += kThreads) {
          const int j = u / wpr;
          const int w = u - j * wpr;
          uint32_t bits = 0;
          if (j < nk) {
            const uint8_t* prow = gpv + size_t(kidx[j]) * N;
            for (int t = 0; t < 32; ++t) {
              const int kk = w * 32 + t;
              if (kk < nk && prow[kidx[kk]] != 0) bits |= 1u << t;
            }
          }
          pvb[j * PW + w] = bits;
        }
      }
    }
    __syncthreads();

    // ---- per-query streaming: one wave owns one query at a time ----
    for (int qs = q0 + wave; qs < q1; qs += kWaves) {
      const int i = qidx[qs];
      const size_t row_off = (size_t(bh) * N + i);

      // q row in fp32, scaled by log2(e), in the GEMM1 B-operand layout:
      // chunk c, element e  <->  d = c*kKPerMfma + g*KPL + e
      float qf[NCH][KPL];
      {
        const T* gq = static_cast<const T*>(p.q) + row_off * D;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int e = 0; e < KPL; ++e) {
            const int d = c * E::kKPerMfma + g * KPL + e;
            qf[c][e] = d < D ? E::to_f32(gq[d]) * kLog2e : 0.0f;
          }
      }

      float M = -INFINITY;  // running max (log2 domain), wave-uniform
      float lsum = 0.0f;    // per-lane partial of sum P
      float acc[NMT][4];
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][r] = 0.0f;

      // optional terms: gates in log2 units, message accumulators
      const bool has_bias = EXT && p.x.u != nullptr;
      const bool has_angle = EXT && p.x.al != nullptr;
      const bool has_msg = EXT == 2 && p.x.ml != nullptr;
      const int a_rank = has_angle ? p.x.a_rank : 0;
      const int m_rank = has_msg ? p.x.m_rank : 0;
      const int a_steps = (a_rank + 3) >> 2;   // 4-wide K steps of the angle MFMA
      const int m_tiles = (m_rank + 15) >> 4;  // 16-row tiles of the message MFMA
      float gq = 0.0f, ga = 0.0f;
      if (has_bias) gq = load_any(p.x.gate, row_off, p.x.bias_dtype) * kLog2e;
      if (has_angle) ga = p.x.ag[row_off] * p.x.a_scale * kLog2e;
      float macc[EXT == 2 ? kRankTiles : 1][4];
#pragma unroll
      for (int rt = 0; rt < (EXT == 2 ? kRankTiles : 1); ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) macc[rt][r] = 0.0f;

      const int njt = ceil_div(nk, 16);
      const int nkc = ceil_div(nk, 64);
      for (int jt = 0; jt < njt; ++jt) {
        const int j = jt * 16 + r16;
        const bool row_ok = j < nk;
        const int jo = row_ok ? kidx[j] : 0;  // original token index of row j

        // per-row terms of this lane's row j
        float uj = 0.0f;
        mf_f32x4 mtacc[EXT == 2 ? kRankTiles : 1];
        if constexpr (EXT) {
          if (has_bias && row_ok) uj = load_any(p.x.u, row_off * N + jo, p.x.bias_dtype);
        }
        if constexpr (EXT == 2) {
#pragma unroll
          for (int rt = 0; rt < kRankTiles; ++rt) mtacc[rt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        }
        // angle B operand source: AL[i][jo][4c + g] (read per use, from L1)
        const float* alrow = EXT && has_angle ? p.x.al + (row_off * N + jo) * a_rank : nullptr;

        // GEMM1 B operand: (q_i (.) k1_j) rounded to the operand type
        typename E::Operand b1[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const T* src = K1s + j * KS + c * E::kKPerMfma + g * KPL;
          if constexpr (KPL == 8) {
            typename E::Operand kv = *reinterpret_cast<const typename E::Operand*>(src);
            typename E::Operand ov;
#pragma unroll
            for (int e = 0; e < 8; ++e) ov[e] = E::from_f32(qf[c][e] * E::to_f32(kv[e]));
            b1[c] = ov;
          } else {
            b1[c] = qf[c][0] * src[0];
          }
        }

        mf_f32x4 tacc[NMT];
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) tacc[mt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};

        for (int kc = 0; kc < nkc; ++kc) {
          const int kbase = kc * 64;
          const int nkt = min(4, ceil_div(nk - kbase, 16));

          // GEMM1: S^T tiles, lane holds row j and keys kbase+kt*16+4g+r
          mf_f32x4 sv[4];
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
            sv[kt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
            if (kt < nkt) {
              const T* arow = K2s + (kbase + kt * 16 + r16) * KS + g * KPL;
#pragma unroll
              for (int c = 0; c < NCH; ++c) {
                typename E::Operand a1;
                if constexpr (KPL == 8) a1 = *reinterpret_cast<const typename E::Operand*>(arow + c * E::kKPerMfma);
                else a1 = arow[c * E::kKPerMfma];
                sv[kt] = E::mma(a1, b1[c], sv[kt]);
              }
            }
          }

          if constexpr (EXT) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
              if (kt >= nkt) continue;
              if (has_angle) {
                // C[k][j] = sum_r AR[i][k][r] AL[i][j][r]: lane supplies A[k = r16][r = 4c + g]
                const int keyA = kbase + kt * 16 + r16;
                const int koA = keyA < nk ? kidx[keyA] : 0;
                const float* arow = p.x.ar + (row_off * N + koA) * a_rank;
                mf_f32x4 at = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < kRankSteps; ++c) {
                  if (c < a_steps) {
                    const int rr = 4 * c + g;
                    const float a = (keyA < nk && rr < a_rank) ? arow[rr] : 0.0f;
                    const float b = (row_ok && rr < a_rank) ? alrow[rr] : 0.0f;
                    at = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, at, 0, 0, 0);
                  }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) sv[kt][r] = fmaf(ga, at[r], sv[kt][r]);
              }
              if (has_bias && row_ok) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const int key = kbase + kt * 16 + 4 * g + r;
                  if (key < nk) {
                    const int ko = kidx[key];
                    const float vk = load_any(p.x.v, row_off * N + ko, p.x.bias_dtype);
                    const float wk = load_any(p.x.w, (size_t(bh) * N + jo) * N + ko, p.x.bias_dtype);
                    sv[kt][r] = fmaf(gq, (uj + vk) + wk, sv[kt][r]);
                  }
                }
              }
            }
          }

          // mask + lane max
          const bool edge = has_pv || (jt * 16 + 16 > nk) || (kbase + nkt * 16 > nk);
          float mloc = -INFINITY;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float sval = sv[kt][r];
              if (kt >= nkt) {
                sval = -INFINITY;
              } else if (edge) {
                const int key = kbase + kt * 16 + 4 * g + r;
                bool ok = row_ok && key < nk;
                if (has_pv && ok) ok = (pvb[j * PW + (key >> 5)] >> (key & 31)) & 1u;
                sval = ok ? sval : -INFINITY;
              }
              sv[kt][r] = sval;
              mloc = fmaxf(mloc, sval);
            }
          }

          // lazy rescale of the running maximum
          if (__any(mloc > M + kRescaleSlack)) {
            const float mw = wave_max(mloc);
            const float Mn = fmaxf(M, mw);
            const float alpha = (M == -INFINITY) ? 0.0f : fast_exp2(M - Mn);
            lsum *= alpha;
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt) {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                acc[mt][r] *= alpha;
                tacc[mt][r] *= alpha;
              }
            }
            if constexpr (EXT == 2) {
              if (has_msg) {
#pragma unroll
                for (int rt = 0; rt < kRankTiles; ++rt)
#pragma unroll
                  for (int r = 0; r < 4; ++r) {
                    macc[rt][r] *= alpha;
                    mtacc[rt][r] *= alpha;
                  }
              }
            }
            M = Mn;
          }
          if (M == -INFINITY) continue;  // nothing valid seen yet

          // P = exp2(S - M)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pe = fast_exp2(sv[kt][r] - M);
              sv[kt][r] = pe;
              lsum += pe;
            }

          // message: CM[r][j] += sum_k MR[i][k][r] P[j][k] (fp32 MFMA; lane
          // supplies A[r = 16 rt + r16][k] for key 4g + rs of tile kt)
          if constexpr (EXT == 2) {
            if (has_msg) {
#pragma unroll
              for (int rt = 0; rt < kRankTiles; ++rt) {
                if (rt >= m_tiles) continue;
                const int rr = 16 * rt + r16;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) {
                  if (kt >= nkt) continue;
#pragma unroll
                  for (int rs = 0; rs < 4; ++rs) {
                    const int key = kbase + kt * 16 + 4 * g + rs;
                    const float a = (key < nk && rr < m_rank) ? p.x.mr[(row_off * N + kidx[key]) * m_rank + rr] : 0.0f;
                    mtacc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, sv[kt][rs], mtacc[rt], 0, 0, 0);
                  }
                }
                // one rank tile's 16 loads in flight at a time (keeps them out of spill range)
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          }

          // GEMM2: C2[d][j] += sum_k V2^T[d][k] P[j][k]
          if constexpr (KPL == 8) {
            using V4 = __attribute__((__vector_size__(4 * sizeof(T)))) T;
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
              if (2 * pr < nkt) {
                typename E::Operand b2;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  b2[r] = E::from_f32(sv[2 * pr][r]);
                  b2[4 + r] = E::from_f32(2 * pr + 1 < nkt ? sv[2 * pr + 1][r] : 0.0f);
                }
                const int kcol = kbase + 32 * pr + 4 * g;
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt) {
                  const T* vrow = V2Ts + (mt * 16 + r16) * VS + kcol;
                  const V4 lo = *reinterpret_cast<const V4*>(vrow);
                  const V4 hi = *reinterpret_cast<const V4*>(vrow + 16);
                  const typename E::Operand a2 = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                  tacc[mt] = E::mma(a2, b2, tacc[mt]);
                }
              }
            }
          } else {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
              if (kt < nkt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const int kcol = kbase + kt * 16 + 4 * g + r;
#pragma unroll
                  for (int mt = 0; mt < NMT; ++mt) {
                    const float a2 = V2Ts[(mt * 16 + r16) * VS + kcol];
                    tacc[mt] = E::mma(a2, sv[kt][r], tacc[mt]);
                  }
                }
              }
            }
          }
        }

        // out_i[d] += sum_j V1[j][d] * C2[d][j]; lane holds j = row, d = mt*16+4g+r.
        // V1 is read from global memory (L1/L2), rows past nk contribute 0.
        if (row_ok) {
          const T* vrow = static_cast<const T*>(p.v1) + (size_t(bh) * N + kidx[j]) * D;
#pragma unroll
          for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int d = mt * 16 + 4 * g + r;
              if (d < D) acc[mt][r] += E::to_f32(vrow[d]) * tacc[mt][r];
            }
        }
        // message: c_r += ML[i][j][r] CM[r][j]; lane holds r = 16 rt + 4g + rr of row j
        if constexpr (EXT == 2) {
          if (has_msg && row_ok) {
            const float* lrow = p.x.ml + (row_off * N + jo) * m_rank;
#pragma unroll
            for (int rt = 0; rt < kRankTiles; ++rt)
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) {
                const int rank = 16 * rt + 4 * g + rr;
                if (rt < m_tiles && rank < m_rank) macc[rt][rr] += lrow[rank] * mtacc[rt][rr];
              }
          }
        }
      }

      // ---- reduce and write the query row ----
      const float lsum_all = wave_sum(lsum);
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][r] = group16_sum(acc[mt][r]);
      const bool has_mass = lsum_all > 0.0f;
      const float inv = has_mass ? 1.0f / lsum_all : 0.0f;
      // message term out[d] += sum_r c_r basis[h][r][d], c_r = Rm^-1/2 * (sum_j CM) / l:
      // after the row-group sum, every lane of group (r & 15) >> 2 holds c_r's sum
      float msg_out[NMT];
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) msg_out[mt] = 0.0f;
      if constexpr (EXT == 2) {
        if (has_msg) {
#pragma unroll
          for (int rt = 0; rt < kRankTiles; ++rt)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) macc[rt][rr] = group16_sum(macc[rt][rr]);
          const float* basis = p.x.mb + size_t(bh % H) * m_rank * D;
          const float cs = p.x.m_scale * inv;
#pragma unroll
          for (int rt = 0; rt < kRankTiles; ++rt) {
            if (rt >= m_tiles) continue;
#pragma unroll
            for (int gs = 0; gs < 4; ++gs)
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) {
                const int r = 16 * rt + 4 * gs + rr;
                const float c = __shfl(macc[rt][rr], 16 * gs, 64) * cs;
                if (r < m_rank) {
#pragma unroll
                  for (int mt = 0; mt < NMT; ++mt) {
                    const int d = mt * 16 + 4 * g + (r16 & 3);
                    if ((mt & 3) == (r16 >> 2) && d < D)
                      msg_out[mt] = fmaf(c, basis[size_t(r) * D + d], msg_out[mt]);
                  }
                }
              }
          }
        }
      }
      // lane (g, r16) writes d = mt*16 + 4g + (r16&3) for mt with (mt&3) == r16>>2
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        if ((mt & 3) != (r16 >> 2)) continue;
        float val = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((r16 & 3) == r) val = acc[mt][r];
        const int d = mt * 16 + 4 * g + (r16 & 3);
        if (d < D) {
          const float o = val * inv + msg_out[mt];
          if (p.out) static_cast<T*>(p.out)[row_off * D + d] = E::from_f32(o);
          if (p.out_f32) p.out_f32[row_off * D + d] = o;
        }
      }
      if (lane == 0 && p.lse)
        p.lse[row_off] = has_mass ? (M + __log2f(lsum_all)) * kLn2 : 0.0f;
    }
    __syncthreads();
  }
}

template <typename T, int DP, int EXT>
int launch(const Params& prm, size_t lds, int grid, hipStream_t stream) {
  auto kern = simplicial_fwd_kernel<T, DP, EXT>;
  constexpr int kThreads = Waves<EXT>::kThreadCount;
  const int st = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), 160 * 1024);
  if (st != MF_OK) return st;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, stream, prm);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

template <typename T>
size_t lds_bytes(int DP, int NP, int B, bool has_pv) {
  switch (DP) {
    case 32: return Layout<T, 32>::bytes(NP, B, has_pv);
    case 64: return Layout<T, 64>::bytes(NP, B, has_pv);
    default: return Layout<T, 128>::bytes(NP, B, has_pv);
  }
}

static size_t lds_for(int dtype, int DP, int NP, int B, bool has_pv) {
  if (dtype == MF_DTYPE_F32) return lds_bytes<float>(DP, NP, B, has_pv);
  if (dtype == MF_DTYPE_F16) return lds_bytes<_Float16>(DP, NP, B, has_pv);
  return lds_bytes<__bf16>(DP, NP, B, has_pv);
}

static int padded_head_dim(int D) { return D <= 32 ? 32 : (D <= 64 ? 64 : 128); }

static int check_shape(int B, int H, int N, int D, int dtype, bool has_pv, size_t* lds_out) {
  if (B <= 0 || H <= 0 || N <= 0 || D <= 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: batch, heads, tokens and head_dim must be positive");
  if (D > 128)
    return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd only supports head_dim <= 128, got " + std::to_string(D));
  if (N > 32767)
    return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd only supports tokens <= 32767");
  if (dtype != MF_DTYPE_F32 && dtype != MF_DTYPE_F16 && dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: unknown dtype " + std::to_string(dtype));
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  const int NP = (N + 31) / 32 * 32;
  const size_t lds = lds_for(dtype, padded_head_dim(D), NP, B, has_pv);
  if (lds > size_t(dev.max_lds_per_block))
    return fail(MF_ERR_UNSUPPORTED,
                "mf_simplicial_fwd: tokens=" + std::to_string(N) + ", head_dim=" + std::to_string(D) +
                    ", batch=" + std::to_string(B) + " needs " + std::to_string(lds) +
                    " bytes of LDS per workgroup, the device offers " + std::to_string(dev.max_lds_per_block));
  if (lds_out) *lds_out = lds;
  return MF_OK;
}

}  // namespace simplicial
}  // namespace mf

using namespace mf;
using namespace mf::simplicial;

// The register-resident kernels take 16-bit operands with head_dim <= 64 and a
// multiple of 8 (whole 16-byte row chunks); everything else, and operands
// that are not 16-byte aligned, runs on the general kernel.
static bool uses_fast(int32_t head_dim, int32_t dtype) {
  return dtype != MF_DTYPE_F32 && head_dim % 8 == 0 && simplicial_fast_capacity(head_dim) > 0;
}

static bool operands_aligned(const mf_simplicial_fwd_args* a) {
  for (const void* ptr : {a->q, a->k1, a->v1, a->k2, a->v2})
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0) return false;
  return true;
}

// ABI 8 operand strides: any set non-zero means a layout other than the contiguous [B*H, N, D].
static bool has_strides(const mf_simplicial_fwd_args* a) {
  for (const int64_t* st : {a->q_stride, a->kv_stride, a->out_stride})
    if (st[0] != 0 || st[1] != 0 || st[2] != 0) return true;
  return false;
}

// Batch stride, in bytes, of a 16-bit operand whose strides are `st` (all zero: contiguous).
static size_t batch_stride_bytes(const int64_t* st, const mf_simplicial_fwd_args* a) {
  if (st[0] == 0 && st[1] == 0 && st[2] == 0) return size_t(a->heads) * a->tokens * a->head_dim * 2;
  return size_t(st[0]) * 2;
}

extern "C" int mf_simplicial_fwd_supported(int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                           int32_t dtype) {
  if (batch <= 0 || heads <= 0 || tokens <= 0 || head_dim <= 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: batch, heads, tokens and head_dim must be positive");
  if (tokens > 32767) return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd only supports tokens <= 32767");
  if (uses_fast(head_dim, dtype)) return MF_OK;
  return check_shape(batch, heads, tokens, head_dim, dtype, /*has_pv=*/true, nullptr);
}

extern "C" uint64_t mf_simplicial_fwd_workspace_size(int32_t batch, int32_t heads, int32_t tokens,
                                                     int32_t head_dim, int32_t dtype) {
  if (batch <= 0 || heads <= 0 || tokens <= 0 || !uses_fast(head_dim, dtype)) return 0;
  // either 16-bit path (unaligned operands take the other one): the pair
  // kernel's claim region first, at the same offset for every shape (its
  // counter stays 0 between calls, so nothing else may write there), then
  // the other kernel's region
  return simplicial_pair_workspace_bytes(batch, tokens) + simplicial_fast_workspace_bytes(batch, heads, tokens);
}

template <int EXT>
static int dispatch(int dtype, int DP, const Params& prm, size_t lds, int grid, hipStream_t s) {
  if (dtype == MF_DTYPE_BF16) {
    if (DP == 32) return launch<__bf16, 32, EXT>(prm, lds, grid, s);
    if (DP == 64) return launch<__bf16, 64, EXT>(prm, lds, grid, s);
    return launch<__bf16, 128, EXT>(prm, lds, grid, s);
  }
  if (dtype == MF_DTYPE_F16) {
    if (DP == 32) return launch<_Float16, 32, EXT>(prm, lds, grid, s);
    if (DP == 64) return launch<_Float16, 64, EXT>(prm, lds, grid, s);
    return launch<_Float16, 128, EXT>(prm, lds, grid, s);
  }
  if (DP == 32) return launch<float, 32, EXT>(prm, lds, grid, s);
  if (DP == 64) return launch<float, 64, EXT>(prm, lds, grid, s);
  return launch<float, 128, EXT>(prm, lds, grid, s);
}

static bool has_extras(const mf_simplicial_fwd_args* a) {
  return a->bias_u != nullptr || a->angle_left != nullptr || a->message_left != nullptr;
}

// Validation of the optional terms (the reference's launcher checks at
// triton_simplicial_attention.py:838-869 and the rank limit of :50-59).
static int check_extras(const mf_simplicial_fwd_args* a) {
  if (a->bias_u || a->bias_v || a->bias_w || a->bias_gate) {
    if (!a->bias_u || !a->bias_v || !a->bias_w || !a->bias_gate)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: bias_u, bias_v, bias_w and bias_gate go together");
    if (a->bias_dtype != MF_DTYPE_F32 && a->bias_dtype != MF_DTYPE_F16 && a->bias_dtype != MF_DTYPE_BF16)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: unknown bias_dtype " + std::to_string(a->bias_dtype));
  }
  if (a->angle_left || a->angle_right || a->angle_gate) {
    if (!a->angle_left || !a->angle_right || !a->angle_gate)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: angle_left, angle_right and angle_gate go together");
    if (a->angle_rank < 1 || a->angle_rank > kMaxRank)
      return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd only supports low-rank features <= 64, got angle rank " +
                                          std::to_string(a->angle_rank));
  }
  if (a->message_left || a->message_right || a->message_basis) {
    if (!a->message_left || !a->message_right || !a->message_basis)
      return fail(MF_ERR_INVALID_ARGUMENT,
                  "mf_simplicial_fwd: message_left, message_right and message_basis go together");
    if (a->message_rank < 1 || a->message_rank > kMaxRank)
      return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd only supports low-rank features <= 64, got message rank " +
                                          std::to_string(a->message_rank));
  }
  return MF_OK;
}

static int launch_general(const mf_simplicial_fwd_args* a, size_t lds, int num_cus, int min_keys, bool zero_rows,
                          hipStream_t s) {
  Params prm{};
  prm.q = a->q; prm.k1 = a->k1; prm.v1 = a->v1; prm.k2 = a->k2; prm.v2 = a->v2;
  prm.qv = a->query_valid; prm.pkv = a->pair_key_valid; prm.pv = a->pair_valid;
  prm.out = a->out; prm.out_f32 = a->out_f32; prm.lse = a->lse;
  prm.B = a->batch; prm.H = a->heads; prm.N = a->tokens; prm.D = a->head_dim;
  prm.NP = (a->tokens + 31) / 32 * 32;
  prm.work_target = 16 * 48 * 48;
  prm.min_keys = min_keys;
  prm.zero_rows = zero_rows ? 1 : 0;
  const size_t esize = a->dtype == MF_DTYPE_F32 ? 4 : 2;
  bool vec = (size_t(a->head_dim) * esize) % 16 == 0;
  for (const void* ptr : {a->q, a->k1, a->v1, a->k2, a->v2})
    vec = vec && (reinterpret_cast<uintptr_t>(ptr) % 16 == 0);
  prm.vec_ok = vec ? 1 : 0;

  const int per_cu = std::max(1, int((160 * 1024) / std::max<size_t>(lds, 1)));
  const int grid = num_cus * std::min(per_cu, 2);
  const int DP = padded_head_dim(a->head_dim);
  if (has_extras(a)) {
    Extras& x = prm.x;
    if (a->bias_u) {
      x.u = a->bias_u; x.v = a->bias_v; x.w = a->bias_w; x.gate = a->bias_gate;
      x.bias_dtype = a->bias_dtype;
    }
    if (a->angle_left) {
      x.al = a->angle_left; x.ar = a->angle_right; x.ag = a->angle_gate;
      x.a_rank = a->angle_rank; x.a_scale = 1.0f / std::sqrt(float(a->angle_rank));
    }
    if (a->message_left) {
      x.ml = a->message_left; x.mr = a->message_right; x.mb = a->message_basis;
      x.m_rank = a->message_rank; x.m_scale = 1.0f / std::sqrt(float(a->message_rank));
    }
    return a->message_left ? dispatch<2>(a->dtype, DP, prm, lds, grid, s)
                           : dispatch<1>(a->dtype, DP, prm, lds, grid, s);
  }
  return dispatch<0>(a->dtype, DP, prm, lds, grid, s);
}

static int simplicial_fwd_impl(const mf_simplicial_fwd_args* a, void* stream);

extern "C" int mf_simplicial_fwd(const mf_simplicial_fwd_args* a, void* stream) {
  return simplicial_fwd_impl(a, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant (for callers that cannot allocate: code under HIP
// graph capture, serving loops).  The scratch the 16-bit kernels need lives
// in this file-scope device array, one copy per GPU, instead of a caller
// workspace.  Host code must not use the array's name as a device address:
// its per-device address comes from hipGetSymbolAddress, taken once per
// device on that device's first call.  Every call on a GPU shares that GPU's
// array, so calls that overlap on one GPU race; each call clears the claim
// counter (the only part that must start at zero) with a fill kernel, which
// stays valid inside captured graphs.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;  // 8 MiB per GPU
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

__global__ void clear_words_kernel(uint32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

static int scratch_address(void** out) {
  static std::mutex mu;
  static std::vector<void*> ptrs;
  int dev = 0;
  MF_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(ptrs.size())) ptrs.resize(dev + 1, nullptr);
  if (ptrs[dev] == nullptr) {
    void* ptr = nullptr;
    MF_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (ptr == nullptr) return fail(MF_ERR_HIP, "mf_simplicial_fwd_noalloc: hipGetSymbolAddress returned NULL");
    ptrs[dev] = ptr;
  }
  *out = ptrs[dev];
  return MF_OK;
}

extern "C" int mf_simplicial_fwd_noalloc(const mf_simplicial_fwd_args* a, void* stream) {
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd_noalloc: args is NULL");
  const uint64_t need =
      mf_simplicial_fwd_workspace_size(a->batch, a->heads, a->tokens, a->head_dim, a->dtype);
  if (need > kNoAllocScratchBytes)
    return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd_noalloc: batch=" + std::to_string(a->batch) +
                                        ", heads=" + std::to_string(a->heads) + ", tokens=" +
                                        std::to_string(a->tokens) + " needs " + std::to_string(need) +
                                        " bytes of scratch, the static scratch holds " +
                                        std::to_string(kNoAllocScratchBytes) + " (use mf_simplicial_fwd)");
  mf_simplicial_fwd_args sub = *a;
  sub.workspace = nullptr;
  sub.workspace_bytes = 0;
  if (need > 0) {
    void* ptr = nullptr;
    int st = scratch_address(&ptr);
    if (st != MF_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int words = int(simplicial_pair_workspace_bytes(a->batch, a->tokens) / 4);
    hipLaunchKernelGGL(clear_words_kernel, dim3(1), dim3(64), 0, s, static_cast<uint32_t*>(ptr), words);
    MF_HIP_CHECK(hipGetLastError());
    sub.workspace = ptr;
    sub.workspace_bytes = kNoAllocScratchBytes;
  }
  return simplicial_fwd_impl(&sub, stream);
}

static int simplicial_fwd_impl(const mf_simplicial_fwd_args* a, void* stream) {
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: args is NULL");
  if (!a->q || !a->k1 || !a->v1 || !a->k2 || !a->v2)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: q, k1, v1, k2 and v2 must be non-NULL");
  if (!a->query_valid || !a->pair_key_valid)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: query_valid and pair_key_valid must be non-NULL");
  if (!a->out && !a->out_f32 && !a->lse)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: at least one of out, out_f32, lse must be non-NULL");
  if (a->precision < MF_PREC_BF16_TC || a->precision > MF_PREC_IEEE_FP32)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: unknown precision " + std::to_string(a->precision));
  if (a->batch <= 0 || a->heads <= 0 || a->tokens <= 0 || a->head_dim <= 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: batch, heads, tokens and head_dim must be positive");
  if (a->dtype != MF_DTYPE_F32 && a->dtype != MF_DTYPE_F16 && a->dtype != MF_DTYPE_BF16)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: unknown dtype " + std::to_string(a->dtype));
  const bool has_pv = a->pair_valid != nullptr;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);

  // 16-bit operands with head_dim <= 64: the register-resident kernels, one
  // set of launches per slice of at most kSimplicialFastMaxBatch molecules
  // (the slices reuse the workspace in stream order).
  st = check_extras(a);
  if (st != MF_OK) return st;
  size_t lds = 0;
  const bool outputs_aligned = reinterpret_cast<uintptr_t>(a->out) % 16 == 0 &&
                               reinterpret_cast<uintptr_t>(a->out_f32) % 16 == 0;
  const bool pair_ok = uses_fast(a->head_dim, a->dtype) && operands_aligned(a) && outputs_aligned &&
                       simplicial_pair_serves(a->tokens, a->head_dim, a->dtype);
  // the factorized bias alone runs in the pair kernel; the angle and message terms (and the bias on
  // other shapes) run on the general kernel
  const bool bias_only = a->bias_u != nullptr && a->angle_left == nullptr && a->message_left == nullptr;
  if (has_strides(a)) {
    if (!pair_ok || has_pv || (has_extras(a) && !bias_only))
      return fail(MF_ERR_UNSUPPORTED,
                  "mf_simplicial_fwd: operand strides other than the contiguous [B*H, N, D] layout are taken by "
                  "the pair kernel only (16-bit operands, head_dim <= 64 and a multiple of 8, tokens <= 512, "
                  "16-byte aligned bases, no pair_valid, no angle or message term)");
    for (const int64_t* st3 : {a->q_stride, a->kv_stride, a->out_stride})
      for (int i = 0; i < 3; ++i)
        if (st3[i] < 0 || st3[i] % 8 != 0)
          return fail(MF_ERR_INVALID_ARGUMENT,
                      "mf_simplicial_fwd: operand strides must be non-negative multiples of 8 elements");
  }
  if (has_extras(a) && !(bias_only && pair_ok)) {
    st = check_shape(a->batch, a->heads, a->tokens, a->head_dim, a->dtype, has_pv, &lds);
    if (st != MF_OK) return st;
    return launch_general(a, lds, dev.num_cus, 0, /*zero_rows=*/true, s);
  }
  if (pair_ok) {
    // the pair-flash kernel: one launch per slice of molecules (the slices
    // share the claim counter at the start of the workspace, in stream order)
    const uint64_t need = simplicial_pair_workspace_bytes(a->batch, a->tokens) +
                          simplicial_fast_workspace_bytes(a->batch, a->heads, a->tokens);
    if (a->workspace == nullptr || a->workspace_bytes < need)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: workspace of " + std::to_string(need) +
                                               " bytes required (mf_simplicial_fwd_workspace_size), got " +
                                               std::to_string(a->workspace_bytes));
    if (reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: workspace must be 16-byte aligned");
    const int slice = simplicial_pair_max_batch(a->tokens);
    const size_t row = size_t(a->heads) * a->tokens;
    const size_t qb = batch_stride_bytes(a->q_stride, a), kvb = batch_stride_bytes(a->kv_stride, a);
    const size_t ob = batch_stride_bytes(a->out_stride, a);
    for (int b0 = 0; b0 < a->batch; b0 += slice) {
      mf_simplicial_fwd_args sub = *a;
      sub.batch = std::min(slice, a->batch - b0);
      sub.q = static_cast<const char*>(a->q) + b0 * qb;
      sub.k1 = static_cast<const char*>(a->k1) + b0 * kvb;
      sub.v1 = static_cast<const char*>(a->v1) + b0 * kvb;
      sub.k2 = static_cast<const char*>(a->k2) + b0 * kvb;
      sub.v2 = static_cast<const char*>(a->v2) + b0 * kvb;
      sub.query_valid = a->query_valid + size_t(b0) * a->tokens;
      sub.pair_key_valid = a->pair_key_valid + size_t(b0) * a->tokens;
      if (a->pair_valid) sub.pair_valid = a->pair_valid + size_t(b0) * a->tokens * a->tokens;
      if (a->out) sub.out = static_cast<char*>(a->out) + b0 * ob;
      if (a->out_f32) sub.out_f32 = a->out_f32 + b0 * row * a->head_dim;
      if (a->lse) sub.lse = a->lse + b0 * row;
      if (a->bias_u) {
        // [B*H, N, N] and [B*H, N] in bias_dtype: the slice's molecules
        const size_t be = a->bias_dtype == MF_DTYPE_F32 ? 4 : 2;
        const size_t pairs = row * a->tokens * be;
        sub.bias_u = static_cast<const char*>(a->bias_u) + b0 * pairs;
        sub.bias_v = static_cast<const char*>(a->bias_v) + b0 * pairs;
        sub.bias_w = static_cast<const char*>(a->bias_w) + b0 * pairs;
        sub.bias_gate = static_cast<const char*>(a->bias_gate) + b0 * row * be;
      }
      st = simplicial_pair_launch(&sub, a->workspace, dev.num_cus, s);
      if (st != MF_OK) return st;
    }
    return MF_OK;
  }
  if (uses_fast(a->head_dim, a->dtype) && operands_aligned(a)) {
    if (a->tokens > 32767) return fail(MF_ERR_UNSUPPORTED, "mf_simplicial_fwd only supports tokens <= 32767");
    // its region follows the pair kernel's claim region
    const uint64_t claims = simplicial_pair_workspace_bytes(a->batch, a->tokens);
    const uint64_t need = claims + simplicial_fast_workspace_bytes(a->batch, a->heads, a->tokens);
    if (a->workspace == nullptr || a->workspace_bytes < need)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: workspace of " + std::to_string(need) +
                                               " bytes required (mf_simplicial_fwd_workspace_size), got " +
                                               std::to_string(a->workspace_bytes));
    if (reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd: workspace must be 16-byte aligned");
    const size_t esize = 2;
    for (int b0 = 0; b0 < a->batch; b0 += kSimplicialFastMaxBatch) {
      mf_simplicial_fwd_args sub = *a;
      const size_t row = size_t(a->heads) * a->tokens;
      const size_t elem = row * a->head_dim * esize;
      sub.batch = std::min(kSimplicialFastMaxBatch, a->batch - b0);
      sub.q = static_cast<const char*>(a->q) + b0 * elem;
      sub.k1 = static_cast<const char*>(a->k1) + b0 * elem;
      sub.v1 = static_cast<const char*>(a->v1) + b0 * elem;
      sub.k2 = static_cast<const char*>(a->k2) + b0 * elem;
      sub.v2 = static_cast<const char*>(a->v2) + b0 * elem;
      sub.query_valid = a->query_valid + size_t(b0) * a->tokens;
      sub.pair_key_valid = a->pair_key_valid + size_t(b0) * a->tokens;
      if (a->pair_valid) sub.pair_valid = a->pair_valid + size_t(b0) * a->tokens * a->tokens;
      if (a->out) sub.out = static_cast<char*>(a->out) + b0 * elem;
      if (a->out_f32) sub.out_f32 = a->out_f32 + b0 * row * a->head_dim;
      if (a->lse) sub.lse = a->lse + b0 * row;
      st = simplicial_fast_launch(&sub, static_cast<char*>(a->workspace) + claims, dev.num_cus, s);
      if (st != MF_OK) return st;
    }
    return MF_OK;
  }
  st = check_shape(a->batch, a->heads, a->tokens, a->head_dim, a->dtype, has_pv, &lds);
  if (st != MF_OK) return st;
  return launch_general(a, lds, dev.num_cus, 0, /*zero_rows=*/true, s);
}

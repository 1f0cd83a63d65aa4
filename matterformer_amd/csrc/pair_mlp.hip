// Factorized simplicial geometry bias in one pass (mf_pair_mlp_bias) on
// gfx950: the three pairwise MLPs of SimplicialGeometryBias
// (src/matterformer/models/transformer.py:566-584,702-717)
//
//   u = MLP_u([delta, rbf(d_norm)]),  v = MLP_v([delta, rbf(d_norm)]),
//   w = MLP_w(rbf(d_norm)),           MLP = Linear -> SiLU -> Linear (H outputs),
//   rbf_r(x) = exp(-gamma (x - c_r)^2)                       (:637-640)
//
// written per head as [B, H, N, N] with the diagonal and the pairs outside
// the geometry pair mask zero (:711-717).  The reference materialises the
// [B, N, N, F] features and the [B, N, N, hidden] activations of each MLP;
// here one wave takes a (molecule b, row i, 64-column group) unit, writes
// the zeros of its invalid pairs, and for each 16-column chunk with a valid
// pair runs the 16 pairs (b, i, j0..j0+15) with everything in registers:
//
//   layer 1  C1[h][p] = b1[h] + sum_f W1[h][f] X[p][f]    fp32 MFMA 16x16x4,
//            M = 16 hidden units, N = 16 pairs, K = 4 features per step;
//            lane (g, r16) computes features g, g+4, ... of pair r16 itself
//   SiLU     on the accumulators
//   layer 2  C2[o][p] = b2[o] + sum_h W2[o][h] SiLU(C1[h][p])
//            the layer-1 accumulators ARE the layer-2 B operands: lane
//            (g, r16) holds hidden units 16 t + 4 g + r of pair r16, so the
//            K step (t, r) takes h = 16 t + 4 g + r with W2 read in the
//            same order
//
// The weights of the three MLPs are staged in LDS once per workgroup (rows
// padded to an odd stride).  fp32 throughout; the exponentials (rbf features,
// SiLU) use the hardware exp2 and reciprocal, a few ulp, well inside the
// rounding of the fp32 sums around them.
#include <algorithm>
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace pmlp {

constexpr int kThreads = 512;  // 8 waves share one copy of the weights
constexpr int kMaxHidden = 256;
constexpr int kMaxHeads = 16;
constexpr int kMaxRbf = 29;  // spoke features 3 + R <= 32

struct Params {
  const float* delta;
  const float* dnorm;
  const uint8_t* mask;
  const float* centers;
  float neg_gamma;
  const float* w1[3];
  const float* b1[3];
  const float* w2[3];
  const float* b2[3];
  float* out[3];
  int B, N, R, hidden, heads, groups;
  // periodic features (PER instantiations): nf Fourier frequencies, the molecule's 6 global features
  int nf;
  const float* freqs;
  const float* glob;
};

__device__ __forceinline__ mf_f32x4 mma(float a, float b, mf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// SiLU x / (1 + e^-x) with the hardware exp2 and reciprocal (about 2 ulp; the fp32 MFMA sums around it carry
// more): e^-x overflows to inf for x < -88, giving -0 as torch's SiLU does
__device__ __forceinline__ float silu(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.44269504088896341f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// One MLP over the 16 pairs of a chunk: layer 1 (K steps of 4 features, x[t] = feature 4 t + g of pair r16),
// SiLU, layer 2; lane (g, r16) returns outputs 4 g .. 4 g + 3 of pair r16.  Two 16-unit hidden slices are
// in flight at a time so one slice's SiLU overlaps the other's MFMA chain.
template <int K>
__device__ __forceinline__ mf_f32x4 mlp16(const float (&x)[K], const float* W1, const float* B1, const float* W2,
                                          const float* B2, int s1, int s2, int HT, int g, int r16) {
  mf_f32x4 o2;
#pragma unroll
  for (int r = 0; r < 4; ++r) o2[r] = B2[4 * g + r];
  const float* w2row = W2 + r16 * s2 + 4 * g;
  int ht = 0;
  for (; ht + 2 <= HT; ht += 2) {
    mf_f32x4 ca, cb;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ca[r] = B1[16 * ht + 4 * g + r];
      cb[r] = B1[16 * ht + 16 + 4 * g + r];
    }
    const float* wa = W1 + (16 * ht + r16) * s1 + g;
    const float* wb = wa + 16 * s1;
#pragma unroll
    for (int t = 0; t < K; ++t) {
      ca = mma(wa[4 * t], x[t], ca);
      cb = mma(wb[4 * t], x[t], cb);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) o2 = mma(w2row[16 * ht + r], silu(ca[r]), o2);
#pragma unroll
    for (int r = 0; r < 4; ++r) o2 = mma(w2row[16 * ht + 16 + r], silu(cb[r]), o2);
  }
  if (ht < HT) {
    mf_f32x4 ca;
#pragma unroll
    for (int r = 0; r < 4; ++r) ca[r] = B1[16 * ht + 4 * g + r];
    const float* wa = W1 + (16 * ht + r16) * s1 + g;
#pragma unroll
    for (int t = 0; t < K; ++t) ca = mma(wa[4 * t], x[t], ca);
#pragma unroll
    for (int r = 0; r < 4; ++r) o2 = mma(w2row[16 * ht + r], silu(ca[r]), o2);
  }
  return o2;
}

// Spoke feature f of a pair under PER (transformer.py:641-652; geometry_bias's _periodic_terms): the delta,
// rbf, then for each delta component c the sines and cosines of (2 pi delta_c) freq_k, then the 6 global
// features of the molecule.
__device__ __forceinline__ float periodic_spoke(const Params& p, int f, float d0, float d1, float d2, float rbf,
                                                int b) {
  const int fb = 3 + p.R, ff = fb + 6 * p.nf;
  if (f < 3) return f == 0 ? d0 : (f == 1 ? d1 : d2);
  if (f < fb) return rbf;
  if (f < ff) {
    const int idx = f - fb, c = idx / (2 * p.nf), rem = idx - c * 2 * p.nf;
    const bool sn = rem < p.nf;
    const float dc = c == 0 ? d0 : (c == 1 ? d1 : d2);
    const float arg = (6.28318530717958647692f * dc) * p.freqs[sn ? rem : rem - p.nf];
    float sv, cv;
    sincosf(arg, &sv, &cv);
    return sn ? sv : cv;
  }
  if (f < ff + 6) return p.glob[size_t(b) * 6 + (f - ff)];
  return 0.0f;
}

// K4: 4-wide K steps of layer 1 for the spoke (u, v) and pair (w) features; PER adds the periodic ones.
template <int KS, int KP, bool PER>
__global__ void __launch_bounds__(kThreads, PER ? 1 : 4) pair_mlp_kernel(Params p) {  // PER: ~128 KB of LDS
  extern __shared__ float lds[];
  const int hidden = p.hidden, H = p.heads;
  const int HT = hidden / 16;
  // per MLP m: W1 [hidden][s1] (K padded with zeros), b1 [hidden], W2 [16][s2] (rows >= H zero), b2 [16]
  const int s1s = 4 * KS + 1, s1p = 4 * KP + 1, s2 = hidden + 1;
  int off[3][4];
  {
    int o = 0;
    for (int m = 0; m < 3; ++m) {
      const int s1 = m < 2 ? s1s : s1p;
      off[m][0] = o;
      o += hidden * s1;
      off[m][1] = o;
      o += hidden;
      off[m][2] = o;
      o += 16 * s2;
      off[m][3] = o;
      o += 16;
    }
  }
  const int tid = threadIdx.x;
  for (int m = 0; m < 3; ++m) {
    const int fin = m < 2 ? 3 + p.R + (PER ? 6 * p.nf + 6 : 0) : p.R + (PER ? 6 : 0);  // true input width
    const int s1 = m < 2 ? s1s : s1p;
    const int kw = 4 * (m < 2 ? KS : KP);
    for (int e = tid; e < hidden * kw; e += kThreads) {
      const int h = e / kw, f = e - h * kw;
      lds[off[m][0] + h * s1 + f] = f < fin ? p.w1[m][h * fin + f] : 0.0f;
    }
    for (int e = tid; e < hidden; e += kThreads) lds[off[m][1] + e] = p.b1[m][e];
    for (int e = tid; e < 16 * hidden; e += kThreads) {
      const int o = e / hidden, h = e - o * hidden;
      lds[off[m][2] + o * s2 + h] = o < H ? p.w2[m][o * hidden + h] : 0.0f;
    }
    for (int e = tid; e < 16; e += kThreads) lds[off[m][3] + e] = e < H ? p.b2[m][e] : 0.0f;
  }
  __syncthreads();

  const int lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int N = p.N, B = p.B;
  const size_t plane = size_t(N) * N;
  // the rbf centres of this lane's features (lane g computes features g, g + 4, ... of its pair)
  const float kexp = p.neg_gamma * 1.44269504088896341f;  // exp(-gamma s) = exp2(kexp s)
  float cs[KS], cp[KP];
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const int f = 4 * t + g;
    cs[t] = (f >= 3 && f < 3 + p.R) ? p.centers[f - 3] : 0.0f;
  }
#pragma unroll
  for (int t = 0; t < KP; ++t) {
    const int f = 4 * t + g;
    cp[t] = f < p.R ? p.centers[f] : 0.0f;
  }
  // unit u = (cg * N + i) * B + b: molecule b, row i, 64-column group cg.  Each lane owns one pair (b, i, j)
  // of the unit and writes the zeros of all outputs when the pair is invalid (256-byte row pieces per
  // store); the 16-column chunks with a valid pair then run the MLPs and write their valid pairs.  Waves
  // take units round-robin, the next unit's (cg, i, b) following by carries (wave-uniform scalar
  // arithmetic), and its pair-mask byte is fetched one unit ahead.
  const int nwaves = gridDim.x * (kThreads / 64);
  const int db = nwaves % B, di = (nwaves / B) % N, dc = (nwaves / B) / N;
  int b, i, cg;
  {
    const int u0 = blockIdx.x * (kThreads / 64) + (tid >> 6);
    b = u0 % B;
    i = (u0 / B) % N;
    cg = (u0 / B) / N;
  }
  auto mask_byte = [&](int bb, int ii, int cc) -> unsigned {
    const int j = cc * 64 + lane;
    if (cc >= p.groups || j >= N) return 0u;
    return p.mask[(size_t(bb) * N + ii) * N + j];
  };
  unsigned mbyte = mask_byte(b, i, cg);
  while (cg < p.groups) {
    int nb = b + db;
    int carry = nb >= B;
    nb -= carry ? B : 0;
    int ni = i + di + carry;
    carry = ni >= N;
    ni -= carry ? N : 0;
    const int ncg = cg + dc + carry;
    const unsigned next = mask_byte(nb, ni, ncg);

    const size_t prow = (size_t(b) * N + i) * N;
    // output element (o, b, i, j): ((b * H + o) * N + i) * N + j
    const size_t obase = size_t(b) * H * plane + size_t(i) * N;
    const int j = cg * 64 + lane;
    const bool in = j < N;
    const bool valid = in && j != i && mbyte != 0u;
    if (in && !valid) {
      for (int m = 0; m < 3; ++m) {
        float* dst = p.out[m] + obase + j;
        for (int o = 0; o < H; ++o) dst[size_t(o) * plane] = 0.0f;
      }
    }
    const unsigned long long bal = __ballot(valid);
    for (int c = 0; c < 4; ++c) {
      const unsigned bits = unsigned(bal >> (16 * c)) & 0xffffu;
      if (bits == 0u) continue;  // wave-uniform
      const int jc = cg * 64 + 16 * c + r16;
      const bool jvalid = (bits >> r16) & 1u;
      const size_t pair = prow + (jvalid ? jc : 0);
      const float dn = jvalid ? p.dnorm[pair] : 0.0f;
      float xs[KS], xp[KP];
      if constexpr (PER) {
        const float d0 = jvalid ? p.delta[3 * pair] : 0.0f;
        const float d1 = jvalid ? p.delta[3 * pair + 1] : 0.0f;
        const float d2 = jvalid ? p.delta[3 * pair + 2] : 0.0f;
#pragma unroll
        for (int t = 0; t < KS; ++t) {
          const float d = dn - cs[t];
          xs[t] = periodic_spoke(p, 4 * t + g, d0, d1, d2, __builtin_amdgcn_exp2f(kexp * (d * d)), b);
        }
#pragma unroll
        for (int t = 0; t < KP; ++t) {
          const int f = 4 * t + g;
          const float d = dn - cp[t];
          xp[t] = f < p.R ? __builtin_amdgcn_exp2f(kexp * (d * d))
                          : (f < p.R + 6 ? p.glob[size_t(b) * 6 + (f - p.R)] : 0.0f);
        }
      } else {
#pragma unroll
        for (int t = 0; t < KS; ++t) {
          const int f = 4 * t + g;
          const float d = dn - cs[t];
          const float rbf = __builtin_amdgcn_exp2f(kexp * (d * d));
          xs[t] = f < 3 ? (jvalid ? p.delta[3 * pair + f] : 0.0f) : (f < 3 + p.R ? rbf : 0.0f);
        }
#pragma unroll
        for (int t = 0; t < KP; ++t) {
          const int f = 4 * t + g;
          const float d = dn - cp[t];
          xp[t] = f < p.R ? __builtin_amdgcn_exp2f(kexp * (d * d)) : 0.0f;
        }
      }
      for (int m = 0; m < 3; ++m) {
        const mf_f32x4 o2 = m < 2 ? mlp16<KS>(xs, lds + off[m][0], lds + off[m][1], lds + off[m][2],
                                               lds + off[m][3], s1s, s2, HT, g, r16)
                                  : mlp16<KP>(xp, lds + off[m][0], lds + off[m][1], lds + off[m][2],
                                              lds + off[m][3], s1p, s2, HT, g, r16);
        if (jvalid) {
          float* dst = p.out[m] + obase + jc;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int o = 4 * g + r;
            if (o < H) dst[size_t(o) * plane] = o2[r];
          }
        }
      }
    }
    b = nb;
    i = ni;
    cg = ncg;
    mbyte = next;
  }
}

size_t lds_bytes(int ks, int kp, int hidden) {
  const size_t s2 = size_t(hidden) + 1;
  size_t floats = 0;
  for (int m = 0; m < 3; ++m) {
    const size_t s1 = 4 * size_t(m < 2 ? ks : kp) + 1;
    floats += size_t(hidden) * s1 + hidden + 16 * s2 + 16;
  }
  return floats * sizeof(float);
}

template <int KS, int KP, bool PER>
int launch(const Params& p, int num_cus, int max_lds, hipStream_t s) {
  const size_t lds = lds_bytes(KS, KP, p.hidden);
  if (lds > size_t(max_lds))
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias: weights exceed the LDS of a workgroup");
  // dynamic LDS above 64 KB needs the attribute (once per kernel and device)
  const int st = ensure_dynamic_lds(reinterpret_cast<const void*>(pair_mlp_kernel<KS, KP, PER>), 160 * 1024);
  if (st != MF_OK) return st;
  const long long units = (long long)p.B * p.N * p.groups;
  const int grid = int(std::min<long long>((units + 7) / 8, (long long)num_cus * 2));
  hipLaunchKernelGGL((pair_mlp_kernel<KS, KP, PER>), dim3(grid), dim3(kThreads), lds, s, p);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

// ---------------------------------------------------------------------------
// Backward (weights): for MLP m over the valid off-diagonal pairs p with upstream gradient dY[o][p]
// (the gradient of the masked output, transformer.py:702-717, so invalid pairs contribute nothing):
//   a1 = W1 x + b1,  h = SiLU(a1),  dH = W2^T dY,  dA = dH (.) SiLU'(a1),  SiLU'(a) = s (1 + a (1 - s)),
//   dW2 += dY h^T,  db2 += dY,  dW1 += dA x^T,  db1 += dA   (db1 as the column of dW1 for a constant-1
//   feature placed after the last real one).
// One workgroup of kBwdThreads takes MLP blockIdx.y; its waves take (molecule, row, 64-column group) units
// as the forward does and, per 16-pair chunk with a valid pair, recompute layer 1 transposed (MFMA 16x16x4
// fp32, pairs as the rows: lane (g, r16) holds pairs 4 g + r of hidden unit r16), form dH^T the same way,
// and accumulate dW1^T [f][h] and dW2 [o][h] by MFMA over the pairs (K): accumulator r of h and dA is the B
// operand of K step r as it is (K index g = pair 4 g + r), so nothing is transposed.  The waves of a workgroup add
// their sums into LDS in wave order and the workgroup writes them to its workspace slot; a second launch adds
// the slots in slot order.  Deterministic (no atomics).
// ---------------------------------------------------------------------------
constexpr int kBwdThreads = 256;
constexpr int kBwdWaves = kBwdThreads / 64;
constexpr int kBwdGroups = 256;     // workgroups per MLP (about three per CU at ~170 registers per lane)
constexpr int kBwdMaxHidden = 128;  // dW1^T / dW2 accumulators in registers: 2 x HT + HT tiles
constexpr int kBwdSlots = kBwdGroups;

struct BwdParams {
  const float* delta;
  const float* dnorm;
  const uint8_t* mask;
  const float* centers;
  float neg_gamma;
  const float* w1[3];
  const float* b1[3];
  const float* w2[3];
  const float* gy[3];   // [B, H, N, N] upstream gradients of u, v, w
  float* dw1[3];        // [hidden, F_m]
  float* db1[3];        // [hidden]
  float* dw2[3];        // [H, hidden]
  float* db2[3];        // [H]
  float* slots;         // [3][kBwdSlots][48 hidden + 16] per-wave partial sums
  int B, N, R, hidden, heads, groups;
};

__host__ __device__ inline size_t bwd_slot_floats(int hidden) { return size_t(48) * hidden + 16; }

template <int KS, int KP>
__global__ void __launch_bounds__(kBwdThreads) pair_mlp_bwd_kernel(BwdParams p) {
  extern __shared__ float lds[];
  const int m = blockIdx.y;
  constexpr int KMAX = KS > KP ? KS : KP;
  const int K = m < 2 ? KS : KP;          // layer-1 K steps (features 4 t + g)
  const int F = m < 2 ? 3 + p.R : p.R;    // true input width; feature F is the constant 1 (db1)
  const int hidden = p.hidden, H = p.heads, HT = hidden / 16;
  const int s1 = 4 * K + 1, s2 = hidden + 1;
  // LDS: W1 [hidden][s1] (columns >= F zero), b1 [hidden], W2 [16][s2] (rows >= H zero), then the
  // workgroup's sums [48 hidden + 16]
  float* W1 = lds;
  float* B1 = W1 + hidden * s1;
  float* W2 = B1 + hidden;
  float* red = W2 + 16 * s2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, r16 = lane & 15;
  for (int e = tid; e < hidden * 4 * K; e += kBwdThreads) {
    const int h = e / (4 * K), f = e - h * (4 * K);
    W1[h * s1 + f] = f < F ? p.w1[m][h * F + f] : 0.0f;
  }
  for (int e = tid; e < hidden; e += kBwdThreads) B1[e] = p.b1[m][e];
  for (int e = tid; e < 16 * hidden; e += kBwdThreads) {
    const int o = e / hidden, h = e - o * hidden;
    W2[o * s2 + h] = o < H ? p.w2[m][o * hidden + h] : 0.0f;
  }
  __syncthreads();

  const int N = p.N, B = p.B;
  const size_t plane = size_t(N) * N;
  const float kexp = p.neg_gamma * 1.44269504088896341f;
  const float* gy = p.gy[m];
  // features of a pair as the layer-1 A operand (feature 4 t + g) and as the dW1 A operand (feature 16 ft + r16)
  const int rb0 = m < 2 ? 3 : 0;  // first rbf feature
  auto feature = [&](size_t pair, float dn, int f) -> float {
    if (f < rb0) return p.delta[3 * pair + f];
    if (f < F) {
      const float d = dn - p.centers[f - rb0];
      return __builtin_amdgcn_exp2f(kexp * (d * d));
    }
    return f == F ? 1.0f : 0.0f;
  };

  mf_f32x4 aw1[2][kBwdMaxHidden / 16], aw2[kBwdMaxHidden / 16];
#pragma unroll
  for (int ht = 0; ht < kBwdMaxHidden / 16; ++ht) {
    aw1[0][ht] = aw1[1][ht] = aw2[ht] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float adb2 = 0.0f;

  const long long units = (long long)B * N * p.groups;
  const int nw = gridDim.x * kBwdWaves;
  for (long long u = (long long)blockIdx.x * kBwdWaves + wave; u < units; u += nw) {
    const int b = int(u % B);
    const int i = int((u / B) % N);
    const int cg = int(u / ((long long)B * N));
    const int j = cg * 64 + lane;
    const bool valid = j < N && j != i && p.mask[(size_t(b) * N + i) * N + min(j, N - 1)] != 0;
    const unsigned long long bal = __ballot(valid);
    const size_t prow = (size_t(b) * N + i) * N;
    for (int c = 0; c < 4; ++c) {
      const unsigned bits = unsigned(bal >> (16 * c)) & 0xffffu;
      if (bits == 0u) continue;  // wave-uniform
      const int j0 = cg * 64 + 16 * c;
      // pair r16 (layer 1, dH): features 4 t + g, upstream gradients of heads 4 s + g
      const bool v16 = (bits >> r16) & 1u;
      const size_t pr = prow + (v16 ? j0 + r16 : 0);
      const float dn16 = v16 ? p.dnorm[pr] : 0.0f;
      float xf[KMAX];
#pragma unroll
      for (int t = 0; t < KMAX; ++t) xf[t] = (t < K && v16) ? feature(pr, dn16, 4 * t + g) : 0.0f;
      float yb[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int o = 4 * s + g;
        yb[s] = (v16 && o < H) ? gy[(size_t(b) * H + o) * plane + size_t(i) * N + j0 + r16] : 0.0f;
      }
      // pairs 4 g + s (dW1 / dW2 A operands of K step s): features 16 ft + r16, upstream gradient of head r16
      float xw[4][2], ya[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int q = 4 * g + s;
        const bool vq = (bits >> q) & 1u;
        const size_t pq = prow + (vq ? j0 + q : 0);
        const float dnq = vq ? p.dnorm[pq] : 0.0f;
#pragma unroll
        for (int ft = 0; ft < 2; ++ft) xw[s][ft] = vq ? feature(pq, dnq, 16 * ft + r16) : 0.0f;
        ya[s] = (vq && r16 < H) ? gy[(size_t(b) * H + r16) * plane + size_t(i) * N + j0 + q] : 0.0f;
        adb2 += ya[s];
      }
      for (int ht = 0; ht < HT; ++ht) {
        // layer 1 and dH, transposed: pairs 4 g + r, hidden unit 16 ht + r16
        const float bias1 = B1[16 * ht + r16];
        mf_f32x4 a1 = mf_f32x4{bias1, bias1, bias1, bias1}, dh = mf_f32x4{0.f, 0.f, 0.f, 0.f};
        const float* wa = W1 + (16 * ht + r16) * s1 + g;
#pragma unroll
        for (int t = 0; t < KMAX; ++t)
          if (t < K) a1 = mma(xf[t], wa[4 * t], a1);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (4 * s < H) dh = mma(yb[s], W2[(4 * s + g) * s2 + 16 * ht + r16], dh);
        float hv[4], dv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = a1[r];
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a * -1.44269504088896341f));
          hv[r] = a * sg;
          dv[r] = dh[r] * (sg * (1.0f + a * (1.0f - sg)));
        }
        // K step s: pairs 4 g + s, i.e. accumulator s of h and dA
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          aw1[0][ht] = mma(xw[s][0], dv[s], aw1[0][ht]);
          aw1[1][ht] = mma(xw[s][1], dv[s], aw1[1][ht]);
          aw2[ht] = mma(ya[s], hv[s], aw2[ht]);
        }
      }
    }
  }
  // the waves' sums added into LDS in wave order: dW1^T [32][hidden] (f = 16 ft + 4 g + r, h = 16 ht + r16),
  // dW2 [16][hidden] (o = 4 g + r), db2 [16] (over the four lane groups); then the workgroup's slot
  adb2 += __shfl_xor(adb2, 16, 64);
  adb2 += __shfl_xor(adb2, 32, 64);
  for (int w = 0; w < kBwdWaves; ++w) {
    if (wave == w) {
      for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int h = 16 * ht + r16;
          float* e0 = red + (4 * g + r) * hidden + h;
          float* e1 = red + (16 + 4 * g + r) * hidden + h;
          float* e2 = red + (32 + 4 * g + r) * hidden + h;
          *e0 = w == 0 ? aw1[0][ht][r] : *e0 + aw1[0][ht][r];
          *e1 = w == 0 ? aw1[1][ht][r] : *e1 + aw1[1][ht][r];
          *e2 = w == 0 ? aw2[ht][r] : *e2 + aw2[ht][r];
        }
      }
      if (g == 0) red[48 * hidden + r16] = w == 0 ? adb2 : red[48 * hidden + r16] + adb2;
    }
    __syncthreads();
  }
  const size_t sf = bwd_slot_floats(hidden);
  float* slot = p.slots + (size_t(m) * kBwdSlots + blockIdx.x) * sf;
  for (int e = tid; e < int(sf); e += kBwdThreads) slot[e] = red[e];
}

// The slots added in slot order, then written as dW1 [hidden][F] (column F of the sums: db1), dW2 [H][hidden],
// db2 [H].
__global__ void __launch_bounds__(256) pair_mlp_bwd_reduce(BwdParams p) {
  const int m = blockIdx.y;
  const int hidden = p.hidden, H = p.heads;
  const int F = m < 2 ? 3 + p.R : p.R;
  const size_t sf = bwd_slot_floats(hidden);
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (size_t(e) >= sf) return;
  const float* src = p.slots + size_t(m) * kBwdSlots * sf + e;
  float s = 0.0f;
  for (int w = 0; w < kBwdSlots; ++w) s += src[size_t(w) * sf];
  if (e < 32 * hidden) {
    const int f = e / hidden, h = e - f * hidden;
    if (f < F) p.dw1[m][h * F + f] = s;
    else if (f == F) p.db1[m][h] = s;
  } else if (e < 48 * hidden) {
    const int o = e / hidden - 32, h = e % hidden;
    if (o < H) p.dw2[m][o * hidden + h] = s;
  } else {
    const int o = e - 48 * hidden;
    if (o < H) p.db2[m][o] = s;
  }
}

}  // namespace pmlp
}  // namespace mf

extern "C" int mf_pair_mlp_bias(const mf_pair_mlp_args* a, void* stream) {
  using namespace mf;
  using namespace mf::pmlp;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias: args is NULL");
  if (!a->pair_delta || !a->pair_dist_norm || !a->pair_mask || !a->rbf_centers)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias: feature pointers must be non-NULL");
  const float* const w1[3] = {a->u_w1, a->v_w1, a->w_w1};
  const float* const b1[3] = {a->u_b1, a->v_b1, a->w_b1};
  const float* const w2[3] = {a->u_w2, a->v_w2, a->w_w2};
  const float* const b2[3] = {a->u_b2, a->v_b2, a->w_b2};
  float* const out[3] = {a->u_out, a->v_out, a->w_out};
  for (int m = 0; m < 3; ++m)
    if (!w1[m] || !b1[m] || !w2[m] || !b2[m] || !out[m])
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias: every weight, bias and output must be non-NULL");
  if (a->batch < 0 || a->atoms < 0) return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias: bad sizes");
  if (a->rbf < 1 || a->rbf > kMaxRbf)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias: rbf features must be in [1, 29]");
  if (a->hidden < 16 || a->hidden > kMaxHidden || a->hidden % 16 != 0)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias: hidden must be a multiple of 16 in [16, 256]");
  if (a->heads < 1 || a->heads > kMaxHeads)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias: heads must be in [1, 16]");
  if (!std::isfinite(a->rbf_gamma)) return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias: gamma must be finite");
  if (a->batch == 0 || a->atoms == 0) return MF_OK;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  Params p{};
  p.delta = a->pair_delta;
  p.dnorm = a->pair_dist_norm;
  p.mask = a->pair_mask;
  p.centers = a->rbf_centers;
  p.neg_gamma = -a->rbf_gamma;
  for (int m = 0; m < 3; ++m) {
    p.w1[m] = w1[m];
    p.b1[m] = b1[m];
    p.w2[m] = w2[m];
    p.b2[m] = b2[m];
    p.out[m] = out[m];
  }
  p.B = a->batch;
  p.N = a->atoms;
  p.R = a->rbf;
  p.hidden = a->hidden;
  p.heads = a->heads;
  p.groups = (a->atoms + 63) / 64;
  if ((long long)a->batch * a->atoms * (p.groups + 1) > 0x7fffffffLL)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias: batch * atoms * ceil(atoms / 64) must stay below 2^31");
  const bool per = a->n_freqs > 0 || a->global_geom != nullptr;
  if (per) {
    if (a->n_freqs < 1 || !a->freqs || !a->global_geom)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias: periodic features need n_freqs >= 1, freqs and "
                                           "global_geom");
    p.nf = a->n_freqs;
    p.freqs = a->freqs;
    p.glob = a->global_geom;
  }
  // spoke K steps (3 + R features, + 6 n_freqs + 6 periodic) and pair K steps (R, + 6 periodic)
  const int ks = (3 + a->rbf + (per ? 6 * a->n_freqs + 6 : 0) + 3) / 4, kp = (a->rbf + (per ? 6 : 0) + 3) / 4;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (per) {
    if (ks > 20 || kp > 9)
      return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias: periodic spoke features must be at most 80 (3 + R + "
                                      "6 n_freqs + 6) and pair features at most 36");
    return launch<20, 9, true>(p, dev.num_cus, dev.max_lds_per_block, s);
  }
  if (ks <= 5 && kp <= 4) return launch<5, 4, false>(p, dev.num_cus, dev.max_lds_per_block, s);
  return launch<8, 8, false>(p, dev.num_cus, dev.max_lds_per_block, s);
}

extern "C" uint64_t mf_pair_mlp_bias_bwd_workspace_size(int32_t hidden) {
  if (hidden < 16 || hidden > mf::pmlp::kBwdMaxHidden || hidden % 16 != 0) return 0;
  return uint64_t(3) * mf::pmlp::kBwdSlots * mf::pmlp::bwd_slot_floats(hidden) * sizeof(float);
}

extern "C" int mf_pair_mlp_bias_bwd(const mf_pair_mlp_bwd_args* a, void* stream) {
  using namespace mf;
  using namespace mf::pmlp;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias_bwd: args is NULL");
  const mf_pair_mlp_args& f = a->fwd;
  if (!f.pair_delta || !f.pair_dist_norm || !f.pair_mask || !f.rbf_centers)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias_bwd: feature pointers must be non-NULL");
  const float* const w1[3] = {f.u_w1, f.v_w1, f.w_w1};
  const float* const b1[3] = {f.u_b1, f.v_b1, f.w_b1};
  const float* const w2[3] = {f.u_w2, f.v_w2, f.w_w2};
  const float* const gy[3] = {a->u_grad, a->v_grad, a->w_grad};
  float* const dw1[3] = {a->u_dw1, a->v_dw1, a->w_dw1};
  float* const db1[3] = {a->u_db1, a->v_db1, a->w_db1};
  float* const dw2[3] = {a->u_dw2, a->v_dw2, a->w_dw2};
  float* const db2[3] = {a->u_db2, a->v_db2, a->w_db2};
  for (int m = 0; m < 3; ++m)
    if (!w1[m] || !b1[m] || !w2[m] || !gy[m] || !dw1[m] || !db1[m] || !dw2[m] || !db2[m])
      return fail(MF_ERR_INVALID_ARGUMENT,
                  "mf_pair_mlp_bias_bwd: every weight, upstream gradient and weight gradient must be non-NULL");
  if (f.batch < 0 || f.atoms < 0) return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias_bwd: bad sizes");
  if (f.n_freqs != 0 || f.global_geom != nullptr)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias_bwd: periodic features are forward-only");
  if (f.rbf < 1 || f.rbf > kMaxRbf - 1)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias_bwd: rbf features must be in [1, 28]");
  if (f.hidden < 16 || f.hidden > kBwdMaxHidden || f.hidden % 16 != 0)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias_bwd: hidden must be a multiple of 16 in [16, 128]");
  if (f.heads < 1 || f.heads > kMaxHeads)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias_bwd: heads must be in [1, 16]");
  if (!std::isfinite(f.rbf_gamma)) return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias_bwd: gamma must be finite");
  const uint64_t need = mf_pair_mlp_bias_bwd_workspace_size(f.hidden);
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_pair_mlp_bias_bwd: workspace smaller than "
                                         "mf_pair_mlp_bias_bwd_workspace_size(hidden)");
  if ((long long)f.batch * f.atoms * ((f.atoms + 63) / 64 + 1) > 0x7fffffffLL)
    return fail(MF_ERR_UNSUPPORTED, "mf_pair_mlp_bias_bwd: batch * atoms * ceil(atoms / 64) must stay below 2^31");
  BwdParams p{};
  p.delta = f.pair_delta;
  p.dnorm = f.pair_dist_norm;
  p.mask = f.pair_mask;
  p.centers = f.rbf_centers;
  p.neg_gamma = -f.rbf_gamma;
  for (int m = 0; m < 3; ++m) {
    p.w1[m] = w1[m]; p.b1[m] = b1[m]; p.w2[m] = w2[m]; p.gy[m] = gy[m];
    p.dw1[m] = dw1[m]; p.db1[m] = db1[m]; p.dw2[m] = dw2[m]; p.db2[m] = db2[m];
  }
  p.slots = static_cast<float*>(a->workspace);
  p.B = f.batch;
  p.N = f.atoms;
  p.R = f.rbf;
  p.hidden = f.hidden;
  p.heads = f.heads;
  p.groups = (f.atoms + 63) / 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int ks = (3 + f.rbf + 1 + 3) / 4, kp = (f.rbf + 1 + 3) / 4;  // K steps holding the features (and F)
  // LDS of the instantiation: W1 rows of 4 KMAX + 1 (the kernel's largest stride), b1, W2, transpose tiles
  auto go = [&](auto kern, int kmax) -> int {
    const size_t lds = (size_t(f.hidden) * (4 * kmax + 1) + f.hidden + 16 * size_t(f.hidden + 1) +
                        bwd_slot_floats(f.hidden)) * sizeof(float);
    const int st = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), int(lds));
    if (st != MF_OK) return st;
    hipLaunchKernelGGL(kern, dim3(kBwdGroups, 3), dim3(kBwdThreads), lds, s, p);
    MF_HIP_CHECK(hipGetLastError());
    const int rblocks = int((bwd_slot_floats(f.hidden) + 255) / 256);
    hipLaunchKernelGGL(pair_mlp_bwd_reduce, dim3(rblocks, 3), dim3(256), 0, s, p);
    MF_HIP_CHECK(hipGetLastError());
    return MF_OK;
  };
  if (ks <= 5 && kp <= 5) return go(pair_mlp_bwd_kernel<5, 5>, 5);
  return go(pair_mlp_bwd_kernel<8, 8>, 8);
}

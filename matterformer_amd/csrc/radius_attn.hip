// Local (radius) attention over a neighbour bit mask (mf_radius_attn) on
// gfx950.
//
// out_i = sum_j softmax_j(scale q_i . k_j over j with mask[i,j]) v_j, the dense
// masked softmax an additive 0/-inf attn_mask gives in nn.MultiheadAttention /
// scaled_dot_product_attention (src/matterformer/models/transformer.py:256-268,
// src/matterformer/models/regular_attention.py:262-268,303-308).  Rows without
// an allowed key give out = 0, lse = 0.
//
// One workgroup (4 waves) per (cell, head, 64-query tile); wave w owns the 16
// queries 16w..16w+15 of the tile.  Key tiles of 64 whose block-mask entry is
// set are staged in LDS (K row-major, V transposed), the next one prefetched
// into registers during the current one's compute.  Per key tile and wave:
//   S^T[key][q] = K Q^T        (MFMA 16x16x32, K rows = A operand from LDS,
//                               Q^T = B operand held in registers)
//   masked online softmax per query column (base 2, scale*log2 e folded in)
//   O^T[d][q]  += V^T P^T      (P^T straight from the S^T accumulators as
//                               the B operand, keys of a 32-key step taken in
//                               the order {4g+r, 16+4g+r}; V^T rows read from
//                               LDS in the same key order)
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace rattn {

constexpr int kThreads = 256;
constexpr int kTile = 64;          // queries per workgroup, keys per tile
constexpr int kMaxTiles = 1024;    // key tiles per row (atoms <= 65536)

struct Params {
  const void* q;
  const void* k;
  const void* v;
  const uint32_t* bits;
  const uint8_t* block_mask;
  void* out;
  float* out_f32;
  float* lse;
  float scale_log2;  // scale * log2(e)
  int B, H, N, W, NB;
  int units;         // B * H * query tiles (the grid is rounded up to a multiple of 8)
};

template <typename T>
struct Ops;
template <>
struct Ops<__bf16> {
  using Op8 = mf_bf16x8;
  __device__ static __forceinline__ mf_f32x4 mma(Op8 a, Op8 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Ops<_Float16> {
  using Op8 = mf_f16x8;
  __device__ static __forceinline__ mf_f32x4 mma(Op8 a, Op8 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T, int D>
__global__ void __launch_bounds__(kThreads) radius_attn_kernel(Params p) {
  using Op8 = typename Ops<T>::Op8;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T Op4;
  constexpr int KS = D + 8;         // K row stride in LDS (elements)
  constexpr int VS = kTile + 8;     // V^T row stride in LDS (elements)
  constexpr int DK = D / 32;        // K steps of S^T
  constexpr int ND = D / 16;        // d tiles of O^T
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  constexpr int CPT = kTile * CPR / kThreads;  // chunks per thread per tile
  static_assert(CPT >= 1 && (kTile * CPR) % kThreads == 0, "staging shape");

  __shared__ __attribute__((aligned(16))) T Ks[2][kTile * KS];  // double-buffered key tiles
  __shared__ __attribute__((aligned(16))) T VT[2][D * VS];
  __shared__ int s_tiles[kMaxTiles];
  __shared__ int s_ntiles;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  // XCD-aware unit order: blockIdx.x % 8 is the XCD, so consecutive logical
  // units -- the query tiles of one (cell, head), which share K and V -- run
  // on one XCD and its L2.
  const int G = gridDim.x;
  const int unit = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  if (unit >= p.units) return;  // grid padding (whole workgroup)
  const int NQT = p.NB;         // query tiles per (cell, head) = key tiles
  const int qt = unit % NQT;
  const int h = (unit / NQT) % p.H;
  const int b = unit / (NQT * p.H);
  const int N = p.N;
  const size_t bh = size_t(b) * p.H + h;
  const T* gq = static_cast<const T*>(p.q) + bh * N * D;
  const T* gk = static_cast<const T*>(p.k) + bh * N * D;
  const T* gv = static_cast<const T*>(p.v) + bh * N * D;

  // active key tiles of this query tile, in order (ballot compaction by wave 0)
  if (wave == 0) {
    const uint8_t* brow = p.block_mask ? p.block_mask + (size_t(b) * p.NB + qt) * p.NB : nullptr;
    int n = 0;
    for (int base = 0; base < p.NB; base += 64) {
      const int jt = base + lane;
      const bool on = jt < p.NB && (!brow || brow[jt] != 0);
      const uint64_t bal = __ballot(on);
      if (on) s_tiles[n + __popcll(bal & ((1ull << lane) - 1))] = jt;
      n += __popcll(bal);
    }
    if (lane == 0) s_ntiles = n;
  }

  // Q^T as B operands: lane holds q = q0 + r16, d = 32 kk + 8 g .. + 7
  const int qi = qt * kTile + wave * 16 + r16;
  const bool q_in = qi < N;
  Op8 qb[DK];
#pragma unroll
  for (int kk = 0; kk < DK; ++kk) {
    if (q_in) {
      qb[kk] = *reinterpret_cast<const Op8*>(gq + size_t(qi) * D + 32 * kk + 8 * g);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[kk][e] = T(0.0f);
    }
  }
  const uint32_t* qbits = p.bits + size_t(b) * N * p.W + size_t(q_in ? qi : 0) * p.W;

  mf_f32x4 acc[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) acc[nd] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  __syncthreads();
  const int ntiles = s_ntiles;

  // register staging of one key tile: chunk c = tid + t*kThreads -> (key c / CPR, d 8*(c % CPR)),
  // and the lane's two mask words of that tile
  // Loads are branch-free (rows past N read row N - 1, mask words past W
  // read word W - 1, and both are zeroed where they are used), so the wait
  // for a tile's loads counts only the loads issued after them.
  struct Stage {
    Op8 k[CPT], v[CPT];
    uint32_t m0, m1;  // mask words as loaded
    uint32_t mok;     // bit 0 / 1: m0 / m1 are real words of a real query
    uint32_t valid;   // bit t: K chunk t is a real key; bit CPT + t: V chunk t
  };
  auto load_tile = [&](int jt, Stage& st) {
    // the words are selected when used (a step later), so that nothing
    // waits for these loads now
    const int w0 = 2 * jt;
    st.m0 = qbits[min(w0, p.W - 1)];
    st.m1 = qbits[min(w0 + 1, p.W - 1)];
    st.mok = (q_in && w0 < p.W ? 1u : 0u) | (q_in && w0 + 1 < p.W ? 2u : 0u);
    st.valid = 0u;
#pragma unroll
    for (int t = 0; t < CPT; ++t) {
      // K: 8 lanes per key row (coalesced); V: 64 consecutive keys per wave
      // and 8-column chunk, so the transposed V^T stores of a wave fill one
      // contiguous row segment
      const int c = tid + t * kThreads;
      const int key = jt * kTile + c / CPR;
      const int d0 = (c % CPR) * 8;
      const int vkey = jt * kTile + c % kTile;
      const int vd0 = (c / kTile) * 8;
      st.k[t] = *reinterpret_cast<const Op8*>(gk + size_t(min(key, N - 1)) * D + d0);
      st.v[t] = *reinterpret_cast<const Op8*>(gv + size_t(min(vkey, N - 1)) * D + vd0);
      st.valid |= (key < N ? 1u << t : 0u) | (vkey < N ? 1u << (CPT + t) : 0u);
    }
  };
  auto store_tile = [&](const Stage& st, int buf) {
#pragma unroll
    for (int t = 0; t < CPT; ++t) {
      const int c = tid + t * kThreads;
      const int key = c / CPR;
      const int d0 = (c % CPR) * 8;
      Op8 kz = st.k[t];
      if (!((st.valid >> t) & 1u)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kz[e] = T(0.0f);
      }
      *reinterpret_cast<Op8*>(Ks[buf] + key * KS + d0) = kz;
      const int vkey = c % kTile;
      const int vd0 = (c / kTile) * 8;
      const bool vok = (st.valid >> (CPT + t)) & 1u;
#pragma unroll
      for (int e = 0; e < 8; ++e) VT[buf][(vd0 + e) * VS + vkey] = vok ? st.v[t][e] : T(0.0f);
    }
  };

  // Tile it is computed from LDS buffer it & 1; tile it + 1 waits in
  // registers and goes to the other buffer at the end of the step; tile it + 2
  // is loaded meanwhile (two tiles of loads in flight, one barrier per tile).
  uint32_t mw0 = 0u, mw1 = 0u;
  Stage sa, sb;
  if (ntiles > 0) {
    load_tile(s_tiles[0], sa);
    if (ntiles > 1) load_tile(s_tiles[1], sb);
    store_tile(sa, 0);
    mw0 = (sa.mok & 1u) ? sa.m0 : 0u;
    mw1 = (sa.mok & 2u) ? sa.m1 : 0u;
    __syncthreads();
  }
  auto step = [&](int it, Stage& freed, const Stage& next) {
    const int buf = it & 1;
    if (it + 2 < ntiles) load_tile(s_tiles[it + 2], freed);
    const T* Kt = Ks[buf];
    const T* VTt = VT[buf];
    // S^T tiles: keys 16 kt + 4 g + r, query r16
    float s[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      mf_f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
        const Op8 a = *reinterpret_cast<const Op8*>(Kt + (16 * kt + r16) * KS + 32 * kk + 8 * g);
        c = Ops<T>::mma(a, qb[kk], c);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) s[kt][r] = c[r];
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = 16 * kt + 4 * g + r;
        const uint32_t word = key < 32 ? mw0 : mw1;
        const bool allowed = (word >> (key & 31)) & 1u;
        s[kt][r] = allowed ? s[kt][r] * p.scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, s[kt][r]);
      }
    }
    // over the 4 key groups g (lanes l ^ 16, l ^ 32): VALU lane swaps
    {
      const auto r16s = __builtin_amdgcn_permlane16_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
      tmax = fmaxf(__uint_as_float(r16s[0]), __uint_as_float(r16s[1]));
      const auto r32s = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
      tmax = fmaxf(__uint_as_float(r32s[0]), __uint_as_float(r32s[1]));
    }
    // The exponent offset m follows the running maximum lazily: it moves
    // only when a logit exceeds it by more than 8 (log2 units), so every
    // p <= 2^8, and the rescaling of the accumulators (MFMA registers) runs
    // only in the rare tiles where some query's offset moves (a wave-uniform
    // branch; the MFMAs need the whole wave).  While a query has seen no
    // allowed key its m stays -inf and its p = exp2(-inf) = 0.
    const bool grow = tmax > m + 8.0f;  // false while tmax is -inf
    if (__ballot(grow) != 0ull) {
      const float m_set = grow ? tmax : m;
      const float alpha = grow ? fast_exp2(m - m_set) : 1.0f;  // 0 when m was -inf
      l *= alpha;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[nd][r] *= alpha;
      }
      m = m_set;
    }
    const float m_off = m == -INFINITY ? 0.0f : m;
    float psum = 0.0f;
    Op8 pb[2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = fast_exp2(s[kt][r] - m_off);  // masked keys: exp2(-inf) = 0
        psum += pv;
        pb[kt >> 1][(kt & 1) * 4 + r] = T(pv);
      }
    }
    l += psum;
    // O^T[d][q] += sum_keys V^T[d][key] P^T[key][q]
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const T* vrow = VTt + (16 * nd + r16) * VS + 32 * pr + 4 * g;
        const Op4 lo = *reinterpret_cast<const Op4*>(vrow);
        const Op4 hi = *reinterpret_cast<const Op4*>(vrow + 16);
        const Op8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[nd] = Ops<T>::mma(a, pb[pr], acc[nd]);
      }
    }
    if (it + 1 < ntiles) store_tile(next, buf ^ 1);
    __syncthreads();
    mw0 = (next.mok & 1u) ? next.m0 : 0u;
    mw1 = (next.mok & 2u) ? next.m1 : 0u;
  };
  for (int it = 0; it < ntiles; it += 2) {
    step(it, sa, sb);
    if (it + 1 < ntiles) step(it + 1, sb, sa);
  }

  // finish: l summed over the 4 key groups g; lane (g, r16) holds d = 16 nd + 4 g + r of query r16
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (!q_in) return;
  const bool has = l > 0.0f;
  const float inv = has ? 1.0f / l : 0.0f;
  const size_t row = bh * N + qi;
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) {
    const int d0 = 16 * nd + 4 * g;
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = acc[nd][r] * inv;
    if (p.out) {
      Op4 ov;
#pragma unroll
      for (int r = 0; r < 4; ++r) ov[r] = T(o[r]);
      *reinterpret_cast<Op4*>(static_cast<T*>(p.out) + row * D + d0) = ov;
    }
    if (p.out_f32) *reinterpret_cast<float4*>(p.out_f32 + row * D + d0) = float4{o[0], o[1], o[2], o[3]};
  }
  if (p.lse && g == 0) p.lse[row] = has ? (m + __log2f(l)) * kLn2 : 0.0f;
}

// ---------------------------------------------------------------------------
// Two key-tile streams (head_dim 32 and 64): 8 waves per (cell, head,
// 64-query tile).  Waves w and w + 4 own the 16 queries 16 (w & 3) .. +15;
// stream e (waves 4e .. 4e + 3) takes the active key tiles of parity e, one
// per step, each staged in LDS by the 256 threads of its stream.  (The
// parity, not the position in the active list, picks the stream, so the
// sums are the same whether or not empty tiles are skipped.)  Per step and wave the work is that of the kernel
// above; with twice the waves per workgroup and half the steps per wave,
// four waves share each SIMD.  At the end the two streams' (O, m, l) of a
// query meet in LDS:
//   out = (2^(m0 - M) O0 + 2^(m1 - M) O1) / (2^(m0 - M) l0 + 2^(m1 - M) l1).
// ---------------------------------------------------------------------------
constexpr int kThreads2 = 512;

// POS: scale > 0.  The running maximum is then taken over the unscaled
// masked logits (scaling preserves the order), p = exp2(s scale - m) is one
// fma per logit, the mask enters as the logit accumulator's start value and
// the row sum is an MFMA with a ones operand.
//
// QW: 16-query tiles per wave (1 or 2).  A workgroup covers 64 QW queries;
// with QW = 2 every K and V operand read from LDS feeds two query tiles (half
// the LDS reads per query), and the workgroup's key tiles are those active in
// either of its two 64-query block rows (a key tile none of a query's keys
// are allowed in adds exactly 0 to that query's sums).
template <typename T, int D, bool POS, int QW>
__global__ void __launch_bounds__(kThreads2, 3 - QW) radius_attn_pair_kernel(Params p) {
  using Op8 = typename Ops<T>::Op8;
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T Op4;
  constexpr int KS = D + 8;         // K row stride in LDS (elements)
  constexpr int DK = D / 32;        // K steps of S^T
  constexpr int ND = D / 16;        // d tiles of O^T
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  constexpr int CPT = kTile * CPR / 256;  // chunks per thread per tile (256 threads per stream)
  static_assert(CPT >= 1 && (kTile * CPR) % 256 == 0, "staging shape");
  static_assert(QW == 1 || QW == 2, "query tiles per wave");
  constexpr int QT = 64 * QW;       // queries per workgroup
  // combine area: QW ND planes of O^T (a float4 per lane of the 4 query
  // groups) and QW planes of (m, l) pairs, consecutive lanes at consecutive
  // addresses (16- and 8-byte LDS accesses without bank conflicts)
  constexpr int kCombBytes = QW * ND * 256 * 16 + QW * 256 * 8;
  static_assert(kCombBytes <= int(sizeof(T)) * 2 * 2 * kTile * KS, "combine area");

  __shared__ __attribute__((aligned(16))) T Ks[2][2][kTile * KS];  // [buffer][stream]
  __shared__ __attribute__((aligned(16))) T Vs[2][2][kTile * KS];  // V row-major, read transposed
  __shared__ int s_tiles[2][kMaxTiles / 2];  // active tiles of each parity, in order
  __shared__ int s_ntiles[2];
  // POS: entry n holds the start of a logit accumulator for mask nibble n
  // (component r: 0 if bit r is set, else -inf)
  __shared__ mf_f32x4 s_lut[16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int kh = wave >> 2, qw = wave & 3;  // key stream, query group
  const int ht = tid & 255;                 // thread index within the stream
  if (POS && tid < 16) {
    mf_f32x4 e;
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = ((tid >> r) & 1) ? 0.0f : -INFINITY;
    s_lut[tid] = e;
  }
  const int G = gridDim.x;
  const int unit = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);  // XCD-aware order
  if (unit >= p.units) return;  // grid padding (whole workgroup)
  const int N = p.N;
  const int NQT = (N + QT - 1) / QT;
  const int qt = unit % NQT;
  const int h = (unit / NQT) % p.H;
  const int b = unit / (NQT * p.H);
  const size_t bh = size_t(b) * p.H + h;
  const T* gq = static_cast<const T*>(p.q) + bh * N * D;
  const T* gk = static_cast<const T*>(p.k) + bh * N * D;
  const T* gv = static_cast<const T*>(p.v) + bh * N * D;

  if (wave < 2) {
    // wave e lists the active tiles of parity e: lane l looks at tile 2 (base + l) + e
    const int br = qt * QW;  // first 64-query block row of the workgroup
    const uint8_t* brow = p.block_mask ? p.block_mask + (size_t(b) * p.NB + br) * p.NB : nullptr;
    const bool two = QW == 2 && br + 1 < p.NB;
    int n = 0;
    for (int base = 0; 2 * base < p.NB; base += 64) {
      const int jt = 2 * (base + lane) + wave;
      bool on = jt < p.NB;
      if (on && brow) on = brow[jt] != 0 || (two && brow[p.NB + jt] != 0);
      const uint64_t bal = __ballot(on);
      if (on) s_tiles[wave][n + __popcll(bal & ((1ull << lane) - 1))] = jt;
      n += __popcll(bal);
    }
    if (lane == 0) s_ntiles[wave] = n;
  }

  int qi[QW];
  bool q_in[QW];
  Op8 qb[QW][DK];
  const uint32_t* qbits[QW];
#pragma unroll
  for (int t = 0; t < QW; ++t) {
    qi[t] = qt * QT + (qw * QW + t) * 16 + r16;
    q_in[t] = qi[t] < N;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk)
      qb[t][kk] = *reinterpret_cast<const Op8*>(gq + size_t(min(qi[t], N - 1)) * D + 32 * kk + 8 * g);
    qbits[t] = p.bits + size_t(b) * N * p.W + size_t(q_in[t] ? qi[t] : 0) * p.W;
  }

  mf_f32x4 acc[QW][ND];
  float m[QW], l[QW];
  // POS: every component of lacc[t] is the sum over the keys seen so far
  mf_f32x4 lacc[QW];
#pragma unroll
  for (int t = 0; t < QW; ++t) {
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc[t][nd] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
    m[t] = -INFINITY;
    l[t] = 0.0f;
    lacc[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  Op8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = T(1.0f);

  __syncthreads();
  const int ntiles = s_ntiles[kh];  // this stream's
  const int nsteps = max(s_ntiles[0], s_ntiles[1]);
  const int* tiles = s_tiles[kh];

  // register staging of this stream's tile of a step (branch-free loads,
  // rows past N zeroed where stored): chunk t of a thread is row c / CPR,
  // columns 8 (c % CPR) (c = ht + 256 t) of both K and V, which are stored
  // row-major alike; offsets within a tile, once
  int krow[CPT], kgo[CPT], kso[CPT];
#pragma unroll
  for (int t = 0; t < CPT; ++t) {
    const int c = ht + t * 256;
    krow[t] = c / CPR;
    kgo[t] = krow[t] * D + (c % CPR) * 8;
    kso[t] = krow[t] * KS + (c % CPR) * 8;
  }
  struct Stage {
    Op8 k[CPT], v[CPT];
    uint32_t m0[QW], m1[QW];  // mask words as loaded
    uint32_t mok[QW];         // bit 0 / 1: m0 / m1 are real words of a real query
    int key0;                 // first key of the tile
    bool full;                // every key of the tile is < N (uniform)
  };
  auto load_tile = [&](int jt, Stage& st) {
    // the words are selected when used (a step later), so that nothing
    // waits for these loads now
    const int w0 = 2 * jt;
#pragma unroll
    for (int t = 0; t < QW; ++t) {
      st.m0[t] = qbits[t][min(w0, p.W - 1)];
      st.m1[t] = qbits[t][min(w0 + 1, p.W - 1)];
      st.mok[t] = (q_in[t] && w0 < p.W ? 1u : 0u) | (q_in[t] && w0 + 1 < p.W ? 2u : 0u);
    }
    const int key0 = jt * kTile;
    st.key0 = key0;
    st.full = key0 + kTile <= N;
    const T* kb = gk + size_t(key0) * D;
    const T* vb = gv + size_t(key0) * D;
    if (st.full) {
#pragma unroll
      for (int t = 0; t < CPT; ++t) {
        st.k[t] = *reinterpret_cast<const Op8*>(kb + kgo[t]);
        st.v[t] = *reinterpret_cast<const Op8*>(vb + kgo[t]);
      }
    } else {
      // rows past N read row N - 1 (zeroed when stored)
#pragma unroll
      for (int t = 0; t < CPT; ++t) {
        const size_t off = size_t(min(key0 + krow[t], N - 1)) * D + (kgo[t] - krow[t] * D);
        st.k[t] = *reinterpret_cast<const Op8*>(gk + off);
        st.v[t] = *reinterpret_cast<const Op8*>(gv + off);
      }
    }
  };
  auto store_tile = [&](const Stage& st, int buf) {
    T* kd = Ks[buf][kh];
    T* vd = Vs[buf][kh];
    if (st.full) {
#pragma unroll
      for (int t = 0; t < CPT; ++t) {
        *reinterpret_cast<Op8*>(kd + kso[t]) = st.k[t];
        *reinterpret_cast<Op8*>(vd + kso[t]) = st.v[t];
      }
    } else {
#pragma unroll
      for (int t = 0; t < CPT; ++t) {
        Op8 kz = st.k[t], vz = st.v[t];
        if (st.key0 + krow[t] >= N) {
#pragma unroll
          for (int e = 0; e < 8; ++e) kz[e] = vz[e] = T(0.0f);
        }
        *reinterpret_cast<Op8*>(kd + kso[t]) = kz;
        *reinterpret_cast<Op8*>(vd + kso[t]) = vz;
      }
    }
  };

  // Step s computes the stream's tile s from buffer s & 1.  The stage holds
  // the loads of step s + 1 (issued after the previous step's store) and
  // goes to the other buffer at the end of the step.
  Stage st;
  uint32_t mw0[QW], mw1[QW];
#pragma unroll
  for (int t = 0; t < QW; ++t) mw0[t] = mw1[t] = 0u;
  auto take_words = [&](const Stage& x) {
#pragma unroll
    for (int t = 0; t < QW; ++t) {
      mw0[t] = (x.mok[t] & 1u) ? x.m0[t] : 0u;
      mw1[t] = (x.mok[t] & 2u) ? x.m1[t] : 0u;
    }
  };
  if (0 < ntiles) {
    load_tile(tiles[0], st);
    store_tile(st, 0);
    take_words(st);
  }
  // Every global load issued so far (q, the first tile) is complete here, on
  // every path.  Were a path to reach the loop with the q loads pending (a
  // stream without tiles), the wait the compiler places before the loop's
  // first use of q would also wait for the next tile's loads, at the start
  // of every step.  (vmcnt(0); expcnt and lgkmcnt unchanged.)
  __builtin_amdgcn_s_waitcnt(0x0F70);
  if (1 < ntiles) load_tile(tiles[1], st);
  __syncthreads();
  const float sc = p.scale_log2;
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    if (s < ntiles) {
      const T* Kt = Ks[buf][kh];
      const T* Vt = Vs[buf][kh];
      float sv[QW][4][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        mf_f32x4 c[QW];
#pragma unroll
        for (int t = 0; t < QW; ++t) {
          // key 16 kt + 4 g + r is bit 16 (kt & 1) + r of (word kt / 2) >> 4 g
          c[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
          if constexpr (POS) c[t] = s_lut[(((kt < 2 ? mw0[t] : mw1[t]) >> (4 * g)) >> (16 * (kt & 1))) & 15u];
        }
#pragma unroll
        for (int kk = 0; kk < DK; ++kk) {
          const Op8 a = *reinterpret_cast<const Op8*>(Kt + (16 * kt + r16) * KS + 32 * kk + 8 * g);
#pragma unroll
          for (int t = 0; t < QW; ++t) c[t] = Ops<T>::mma(a, qb[t][kk], c[t]);
        }
#pragma unroll
        for (int t = 0; t < QW; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[t][kt][r] = c[t][r];
      }
      Op8 pb[QW][2];
#pragma unroll
      for (int t = 0; t < QW; ++t) {
        float tmax = -INFINITY;
        if constexpr (POS) {
          // this lane's maximum only; the query's (over its 4 lanes) is
          // formed when some lane of the wave may move its offset
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sv[t][kt][r]);
          tmax *= sc;  // -inf stays -inf
          if (__ballot(tmax > m[t] + 8.0f) != 0ull) {
            const auto r16s = __builtin_amdgcn_permlane16_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
            tmax = fmaxf(__uint_as_float(r16s[0]), __uint_as_float(r16s[1]));
            const auto r32s = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
            tmax = fmaxf(__uint_as_float(r32s[0]), __uint_as_float(r32s[1]));
            const bool grow = tmax > m[t] + 8.0f;  // the same for the 4 lanes of a query
            const float m_set = grow ? tmax : m[t];
            const float alpha = grow ? fast_exp2(m[t] - m_set) : 1.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) lacc[t][r] *= alpha;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[t][nd][r] *= alpha;
            m[t] = m_set;
          }
        } else {
          const uint32_t wa = mw0[t] >> (4 * g), wb = mw1[t] >> (4 * g);
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const bool allowed = (((kt < 2 ? wa : wb) >> (16 * (kt & 1) + r)) & 1u) != 0u;
              sv[t][kt][r] = allowed ? sv[t][kt][r] * sc : -INFINITY;
              tmax = fmaxf(tmax, sv[t][kt][r]);
            }
          }
          const auto r16s = __builtin_amdgcn_permlane16_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
          tmax = fmaxf(__uint_as_float(r16s[0]), __uint_as_float(r16s[1]));
          const auto r32s = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
          tmax = fmaxf(__uint_as_float(r32s[0]), __uint_as_float(r32s[1]));
          // lazy offset, as in the kernel above
          const bool grow = tmax > m[t] + 8.0f;
          if (__ballot(grow) != 0ull) {
            const float m_set = grow ? tmax : m[t];
            const float alpha = grow ? fast_exp2(m[t] - m_set) : 1.0f;
            l[t] *= alpha;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[t][nd][r] *= alpha;
            m[t] = m_set;
          }
        }
        const float m_off = m[t] == -INFINITY ? 0.0f : m[t];
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pv = POS ? fast_exp2(fmaf(sv[t][kt][r], sc, -m_off)) : fast_exp2(sv[t][kt][r] - m_off);
            if constexpr (!POS) psum += pv;
            pb[t][kt >> 1][(kt & 1) * 4 + r] = T(pv);
          }
        }
        if constexpr (POS) {
          lacc[t] = Ops<T>::mma(ones, pb[t][0], lacc[t]);
          lacc[t] = Ops<T>::mma(ones, pb[t][1], lacc[t]);
        } else {
          l[t] += psum;
        }
      }
      // V^T operands straight from the row-major tile: within each group of
      // 16 lanes, ds_read_b64_tr_b16 hands lane 4a + c element c of the
      // 8-byte pieces addressed by lanes 4e + a (e = 0..3).  Lane 4e + a
      // addresses key 32 pr + 4 g + e (+16 for the second read), columns
      // 16 nd + 4a .. +3, so lane r16 receives V[keys 32 pr + 4 g + 0..3]
      // [d = 16 nd + r16]: the key order of the P^T operand.
      const T* vt0 = Vt + (4 * g + (r16 >> 2)) * KS + 4 * (r16 & 3);
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const T* vp = vt0 + 32 * pr * KS + 16 * nd;
          const Op4 lo = read_tr16<T>(vp);
          const Op4 hi = read_tr16<T>(vp + 16 * KS);
          const Op8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
          for (int t = 0; t < QW; ++t) acc[t][nd] = Ops<T>::mma(a, pb[t][pr], acc[t][nd]);
        }
      }
    }
    if (s + 1 < ntiles) {
      store_tile(st, buf ^ 1);
      take_words(st);
    }
    __syncthreads();
    if (s + 2 < ntiles) load_tile(tiles[s + 2], st);
  }

  // combine the streams: l summed over the 4 key groups g first (POS: the
  // MFMA row sum already holds every key)
#pragma unroll
  for (int t = 0; t < QW; ++t) {
    if constexpr (POS) {
      l[t] = lacc[t][0];
    } else {
      l[t] += __shfl_xor(l[t], 16, 64);
      l[t] += __shfl_xor(l[t], 32, 64);
    }
  }
  // (after the last barrier: the K tiles are no longer read)
  mf_f32x4* cmb_o = reinterpret_cast<mf_f32x4*>(&Ks[0][0][0]);  // [QW][ND][4 query groups x 64 lanes]
  float2* cmb_ml = reinterpret_cast<float2*>(cmb_o + QW * ND * 256);  // [QW][4 x 64]
  const int slot = qw * 64 + lane;
  if (kh == 1) {
#pragma unroll
    for (int t = 0; t < QW; ++t) {
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) cmb_o[(t * ND + nd) * 256 + slot] = acc[t][nd];
      cmb_ml[t * 256 + slot] = float2{m[t], l[t]};
    }
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int t = 0; t < QW; ++t) {
    if (!q_in[t]) continue;
    const float2 ml = cmb_ml[t * 256 + slot];
    const float m1 = ml.x, l1 = ml.y;
    const float M = fmaxf(m[t], m1);
    const float a0 = M == -INFINITY ? 0.0f : fast_exp2(m[t] - M);  // 0 for a stream without allowed keys
    const float a1 = M == -INFINITY ? 0.0f : fast_exp2(m1 - M);
    const float L = a0 * l[t] + a1 * l1;
    const bool has = L > 0.0f;
    const float inv = has ? 1.0f / L : 0.0f;
    const size_t row = bh * N + qi[t];
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      const int d0 = 16 * nd + 4 * g;
      const mf_f32x4 c1 = cmb_o[(t * ND + nd) * 256 + slot];
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (a0 * acc[t][nd][r] + a1 * c1[r]) * inv;
      if (p.out) {
        Op4 ov;
#pragma unroll
        for (int r = 0; r < 4; ++r) ov[r] = T(o[r]);
        *reinterpret_cast<Op4*>(static_cast<T*>(p.out) + row * D + d0) = ov;
      }
      if (p.out_f32) *reinterpret_cast<float4*>(p.out_f32 + row * D + d0) = float4{o[0], o[1], o[2], o[3]};
    }
    if (p.lse && g == 0) p.lse[row] = has ? (M + __log2f(L)) * kLn2 : 0.0f;
  }
}

template <typename T, int D>
int launch(const Params& p, hipStream_t stream) {
  const dim3 grid((p.units + 7) / 8 * 8);
  hipLaunchKernelGGL((radius_attn_kernel<T, D>), grid, dim3(kThreads), 0, stream, p);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

// Two query tiles per wave once a (cell, head) spans more than three 64-query
// tiles (the 128-query workgroups then waste at most a quarter of a tile's
// queries to padding) and the launch still has a workgroup per CU.
template <typename T, int D>
int launch_pair(const Params& p, hipStream_t stream) {
  const bool wide = p.N > 3 * kTile && (long long)p.B * p.H * ((p.N + 2 * kTile - 1) / (2 * kTile)) >= 256;
  Params q = p;
  if (wide) q.units = p.B * p.H * ((p.N + 2 * kTile - 1) / (2 * kTile));
  const dim3 grid((q.units + 7) / 8 * 8);
  if (p.scale_log2 > 0.0f) {
    if (wide) hipLaunchKernelGGL((radius_attn_pair_kernel<T, D, true, 2>), grid, dim3(kThreads2), 0, stream, q);
    else hipLaunchKernelGGL((radius_attn_pair_kernel<T, D, true, 1>), grid, dim3(kThreads2), 0, stream, q);
  } else {
    if (wide) hipLaunchKernelGGL((radius_attn_pair_kernel<T, D, false, 2>), grid, dim3(kThreads2), 0, stream, q);
    else hipLaunchKernelGGL((radius_attn_pair_kernel<T, D, false, 1>), grid, dim3(kThreads2), 0, stream, q);
  }
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

template <typename T>
int dispatch_dim(const Params& p, int D, hipStream_t stream) {
  if (D == 32) return launch_pair<T, 32>(p, stream);
  if (D == 64) return launch_pair<T, 64>(p, stream);
  return launch<T, 128>(p, stream);
}

}  // namespace rattn
}  // namespace mf

extern "C" int mf_radius_attn(const mf_radius_attn_args* a, void* stream) {
  using namespace mf;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_attn: args is NULL");
  if (!a->q || !a->k || !a->v || !a->mask_bits)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_attn: q, k, v and mask_bits must be non-NULL");
  if (!a->out && !a->out_f32 && !a->lse)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_attn: at least one of out, out_f32, lse must be non-NULL");
  if (a->batch < 0 || a->heads < 0 || a->atoms < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_attn: batch, heads and atoms must be non-negative");
  if (a->dtype != MF_DTYPE_BF16 && a->dtype != MF_DTYPE_F16)
    return fail(MF_ERR_UNSUPPORTED, "mf_radius_attn: only supports float16/bfloat16 operands");
  if (a->head_dim != 32 && a->head_dim != 64 && a->head_dim != 128)
    return fail(MF_ERR_UNSUPPORTED, "mf_radius_attn: head_dim must be 32, 64 or 128");
  if (!std::isfinite(a->scale)) return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_attn: scale must be finite");
  for (const void* ptr : {a->q, a->k, a->v, static_cast<const void*>(a->out), static_cast<const void*>(a->out_f32)})
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0)
      return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_attn: q, k, v, out and out_f32 must be 16-byte aligned");
  if (a->batch == 0 || a->heads == 0 || a->atoms == 0) return MF_OK;
  const int nb = (a->atoms + rattn::kTile - 1) / rattn::kTile;
  if (nb > rattn::kMaxTiles) return fail(MF_ERR_UNSUPPORTED, "mf_radius_attn: atoms must be <= 65536");
  const long long units = (long long)a->batch * a->heads * nb;
  if (units > 0x7fffffffLL - 8) return fail(MF_ERR_UNSUPPORTED, "mf_radius_attn: batch * heads * tiles too large");
  rattn::Params p{a->q, a->k, a->v, a->mask_bits, a->block_mask, a->out, a->out_f32, a->lse,
                  a->scale * kLog2e, a->batch, a->heads, a->atoms, (a->atoms + 31) / 32, nb, int(units)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == MF_DTYPE_BF16) return rattn::dispatch_dim<__bf16>(p, a->head_dim, s);
  return rattn::dispatch_dim<_Float16>(p, a->head_dim, s);
}

// k nearest neighbours of every atom of a batch of molecules (mf_knn) on
// gfx950.
//
// Distances follow NonPeriodicGeometryAdapter.forward
// (src/matterformer/geometry/adapters.py:98-100): delta = x_i - x_j,
// d2 = (dx*dx + dy*dy) + dz*dz in fp32 with every operation rounded (this file
// is built with -ffp-contract=off, so no FMA is formed).  The order is the
// stable one, (d2, j) ascending, which the legacy torch_cluster / topk path
// (legacy/rapidash_v5/models/rapidash_utils.py:139-193) leaves unspecified.
//
// Layout: one workgroup of 256 threads serves 256/L queries of one molecule;
// the L lanes of a query split the candidates j (lane s takes j = s mod L),
// reading the molecule's coordinates from LDS tiles of kTile atoms (every lane
// of a wave reads the same few words per step: broadcast, no bank conflicts).
// Each lane keeps the KMAX smallest keys it has seen, sorted, in registers:
//   key = float_bits(d2) << 32 | j
// (d2 >= 0, so the float bit pattern orders like the value and the low word
// breaks ties by index).
//   k <= 16 (knn_block_kernel): a lane takes its candidates KMAX at a time:
//     the block's keys are sorted by a bitonic network and merged into the
//     list as min(list[s], block[KMAX-1-s]) (a bitonic sequence holding the
//     KMAX smallest of both) followed by a bitonic clean-up; a block none of
//     whose keys is below the wave's current KMAX-th keys is skipped.  No
//     step depends on the data, so the 64 lanes of a wave never diverge (an
//     insertion chain runs for the wave whenever one lane inserts, which is
//     nearly every candidate).
//   k > 16 (knn_kernel): a candidate below the current KMAX-th key is merged
//     in by one compare-exchange chain.
// The L lists of a query are then merged in log2(L) butterfly rounds:
// partners exchange lists, take min(a[s], b[KMAX-1-s]) and clean up with the
// bitonic network, so both partners end with the same list.
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace knn {

constexpr int kThreads = 256;
constexpr int kTile = 2048;  // atoms staged in LDS per pass (24 KB + 2 KB)
constexpr uint64_t kEmpty = ~0ull;

struct Params {
  const float* coords;
  const uint8_t* pad;
  int32_t* idx;
  float* dist;
  int B, N, K, exclude_self;
};

// One 64-bit compare per comparator: the maximum is the other key,
// a ^ b ^ min(a, b) (exact for equal keys too), so the compiler does not
// expand a separate umax with a second compare.
__device__ __forceinline__ void cmp_swap(uint64_t& lo, uint64_t& hi) {
  const uint64_t a = lo, b = hi;
  const uint64_t mn = a < b ? a : b;
  // v_bitop3_b32 with truth table 0x96 is the 3-input XOR
  const uint32_t h0 = __builtin_amdgcn_bitop3_b32(uint32_t(a), uint32_t(b), uint32_t(mn), 0x96);
  const uint32_t h1 = __builtin_amdgcn_bitop3_b32(uint32_t(a >> 32), uint32_t(b >> 32), uint32_t(mn >> 32), 0x96);
  hi = (uint64_t(h1) << 32) | h0;
  lo = mn;
}

// 32-bit keys (knn_code_kernel): a plain min / max pair.
__device__ __forceinline__ void cmp_swap(uint32_t& lo, uint32_t& hi) {
  const uint32_t a = lo, b = hi;
  lo = a < b ? a : b;
  hi = a < b ? b : a;
}

template <int KMAX>
__device__ __forceinline__ void insert(uint64_t (&list)[KMAX], uint64_t key) {
#pragma unroll
  for (int s = 0; s < KMAX; ++s) cmp_swap(list[s], key);
}

// Sort a bitonic sequence ascending.
template <typename Key, int KMAX>
__device__ __forceinline__ void bitonic_sort(Key (&list)[KMAX]) {
#pragma unroll
  for (int stride = KMAX / 2; stride >= 1; stride >>= 1) {
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if ((s & stride) == 0) cmp_swap(list[s], list[s + stride]);
  }
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), mask, 64);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), mask, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Sort KMAX keys ascending: Batcher's odd-even merge sort (K. E. Batcher,
// "Sorting networks and their applications", AFIPS 1968), 63 comparators for
// 16 keys and 19 for 8 (a bitonic sorting network takes 80 and 24).
// oe_merge merges the sorted halves of v[LO .. LO + N) taken with stride R.
template <int KMAX, int LO, int N, int R, typename Key>
__device__ __forceinline__ void oe_merge(Key (&v)[KMAX]) {
  constexpr int kStep = 2 * R;
  if constexpr (kStep < N) {
    oe_merge<KMAX, LO, N, kStep>(v);
    oe_merge<KMAX, LO + R, N, kStep>(v);
#pragma unroll
    for (int i = LO + R; i < LO + N - R; i += kStep) cmp_swap(v[i], v[i + R]);
  } else {
    cmp_swap(v[LO], v[LO + R]);
  }
}
template <int KMAX, int LO, int N, typename Key>
__device__ __forceinline__ void oe_sort(Key (&v)[KMAX]) {
  if constexpr (N > 1) {
    oe_sort<KMAX, LO, N / 2>(v);
    oe_sort<KMAX, LO + N / 2, N / 2>(v);
    oe_merge<KMAX, LO, N, 1>(v);
  }
}

// The 64-bit value of the partner lane in a butterfly merge over groups of
// consecutive lanes: quad permutes for masks 1 and 2, then the half-row and
// row mirrors (lane l of an 8 / 16 group meets the lane at the mirrored
// position of the other half; after the earlier rounds every lane of a half
// holds the same list, so any cross pairing merges the two halves).
template <int MASK>
__device__ __forceinline__ uint32_t partner_u32(uint32_t v) {
  constexpr int ctrl = MASK == 1 ? 0xB1 : MASK == 2 ? 0x4E : MASK == 4 ? 0x141 : 0x140;
  static_assert(MASK == 1 || MASK == 2 || MASK == 4 || MASK == 8, "lanes per query <= 16");
  return uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), ctrl, 0xf, 0xf, false));
}
template <int MASK>
__device__ __forceinline__ uint64_t partner_u64(uint64_t v) {
  return (uint64_t(partner_u32<MASK>(uint32_t(v >> 32))) << 32) | partner_u32<MASK>(uint32_t(v));
}
template <int MASK>
__device__ __forceinline__ uint64_t partner(uint64_t v) { return partner_u64<MASK>(v); }
template <int MASK>
__device__ __forceinline__ uint32_t partner(uint32_t v) { return partner_u32<MASK>(v); }

// One butterfly round per lane-count doubling.  With TRACK, out_min also
// collects the smallest key either partner let go (its own and the other's
// running minimum, and the larger of every min(a[s], b[KMAX-1-s]) pair).
template <int KMAX, int L, int MASK, bool TRACK = false, typename Key>
__device__ __forceinline__ void merge_round(Key (&list)[KMAX], Key& out_min) {
  if constexpr (MASK < L) {
    Key other[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s) other[s] = partner<MASK>(list[KMAX - 1 - s]);
    if constexpr (TRACK) {
      const Key o = partner<MASK>(out_min);
      out_min = out_min < o ? out_min : o;
    }
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      const Key a = list[s], b = other[s];
      list[s] = a < b ? a : b;
      if constexpr (TRACK) {
        const Key hi = a < b ? b : a;
        out_min = out_min < hi ? out_min : hi;
      }
    }
    bitonic_sort(list);
    merge_round<KMAX, L, MASK * 2, TRACK>(list, out_min);
  }
}

template <int KMAX, int L>
__global__ void __launch_bounds__(kThreads) knn_block_kernel(Params p) {
  __shared__ float sx[kTile], sy[kTile], sz[kTile];
  __shared__ uint8_t spad[kTile];

  constexpr int kQueries = kThreads / L;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int sub = tid % L;
  const int i = blockIdx.x * kQueries + tid / L;
  const int N = p.N;
  const float* x = p.coords + size_t(b) * N * 3;
  const uint8_t* pad = p.pad ? p.pad + size_t(b) * N : nullptr;
  const bool valid_i = i < N && !(pad && pad[i]);
  float xi = 0.0f, yi = 0.0f, zi = 0.0f;
  if (valid_i) {
    xi = x[3 * i + 0];
    yi = x[3 * i + 1];
    zi = x[3 * i + 2];
  }

  uint64_t list[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) list[s] = kEmpty;

  for (int t0 = 0; t0 < N; t0 += kTile) {
    const int n = min(kTile, N - t0);
    __syncthreads();
    for (int u = tid; u < n; u += kThreads) {
      sx[u] = x[3 * (t0 + u) + 0];
      sy[u] = x[3 * (t0 + u) + 1];
      sz[u] = x[3 * (t0 + u) + 2];
      spad[u] = pad ? pad[t0 + u] : 0;
    }
    __syncthreads();
    // every lane runs the same number of blocks (invalid queries see only
    // empty keys), so the whole wave stays converged
    for (int u0 = sub; u0 - sub < n; u0 += L * KMAX) {
      uint64_t blk[KMAX];
      bool below = false;
#pragma unroll
      for (int t = 0; t < KMAX; ++t) {
        const int u = u0 + L * t;
        const int j = t0 + u;
        uint64_t key = kEmpty;
        if (valid_i && u < n && !spad[u] && !(p.exclude_self && j == i)) {
          const float dx = xi - sx[u];
          const float dy = yi - sy[u];
          const float dz = zi - sz[u];
          const float xx = dx * dx;
          const float yy = dy * dy;
          const float zz = dz * dz;
          const float s2 = xx + yy;
          const float d2 = s2 + zz;
          key = (static_cast<uint64_t>(__float_as_uint(d2)) << 32) | static_cast<uint32_t>(j);
        }
        blk[t] = key;
        below |= key < list[KMAX - 1];
      }
      if (!__any(below)) continue;  // no lane of the wave keeps any of these
      oe_sort<KMAX, 0, KMAX>(blk);
#pragma unroll
      for (int s = 0; s < KMAX; ++s) list[s] = list[s] < blk[KMAX - 1 - s] ? list[s] : blk[KMAX - 1 - s];
      bitonic_sort(list);
    }
  }

  uint64_t unused = 0;
  merge_round<KMAX, L, 1>(list, unused);

  if (i >= N) return;
  int32_t* oi = p.idx + (size_t(b) * N + i) * p.K;
  float* od = p.dist ? p.dist + (size_t(b) * N + i) * p.K : nullptr;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s % L != sub || s >= p.K) continue;
    const uint64_t key = list[s];
    const bool empty = key == kEmpty;
    oi[s] = empty ? -1 : static_cast<int32_t>(static_cast<uint32_t>(key));
    if (od) od[s] = empty ? INFINITY : sqrtf(__uint_as_float(static_cast<uint32_t>(key >> 32)));
  }
}

// ---------------------------------------------------------------------------
// Molecules of at most kCodeAtoms atoms, k <= 16: 32-bit keys.
//
//   code = (float_bits(d2) >> 7) << 8 | j        (j < 256)
//
// orders like (d2, j) except among keys whose d2 agree in all but the 7
// lowest mantissa bits (relative difference < 2^-16), which it orders by j.
// A comparator on these keys is one v_min_u32 and one v_max_u32 instead of
// a 64-bit compare and four selects, so the block sort and merge cost less
// than half.  Exactness is restored per query at the end:
//   * every key a lane drops (the larger of each min(list[s], blk[K-1-s])
//     pair, the blocks it skips, the butterfly's losers) is folded into
//     out_min, the smallest key outside the list;
//   * if the k-th key's d2 code is strictly below that of the next key
//     (list[k] for k < KMAX, else out_min), the k kept atoms are exactly the
//     k smallest by (d2, j) -- every key outside has a larger d2 -- and only
//     their order may differ: their exact d2 is recomputed and they are
//     re-sorted with 64-bit keys;
//   * otherwise (a code shared across the boundary: duplicate atoms, or d2
//     equal to 2^-16) the query is recomputed with the 64-bit block scan.
// ---------------------------------------------------------------------------
constexpr int kCodeAtoms = 256;
constexpr uint32_t kEmpty32 = ~0u;

__device__ __forceinline__ float pair_d2(float xi, float yi, float zi, float xj, float yj, float zj) {
  const float dx = xi - xj;
  const float dy = yi - yj;
  const float dz = zi - zj;
  const float xx = dx * dx;
  const float yy = dy * dy;
  const float zz = dz * dz;
  const float s2 = xx + yy;
  return s2 + zz;
}

// The 64-bit block scan over the atoms staged in LDS (the whole molecule).
template <int KMAX, int L>
__device__ __forceinline__ void exact_scan(uint64_t (&list)[KMAX], const float* sx, const float* sy, const float* sz,
                                           const uint8_t* spad, int n, int i, int sub, bool valid_i,
                                           int exclude_self, float xi, float yi, float zi) {
#pragma unroll
  for (int s = 0; s < KMAX; ++s) list[s] = kEmpty;
  for (int u0 = sub; u0 - sub < n; u0 += L * KMAX) {
    uint64_t blk[KMAX];
    bool below = false;
#pragma unroll
    for (int t = 0; t < KMAX; ++t) {
      const int u = u0 + L * t;
      uint64_t key = kEmpty;
      if (valid_i && u < n && !spad[u] && !(exclude_self && u == i))
        key = (static_cast<uint64_t>(__float_as_uint(pair_d2(xi, yi, zi, sx[u], sy[u], sz[u]))) << 32) | uint32_t(u);
      blk[t] = key;
      below |= key < list[KMAX - 1];
    }
    if (!__any(below)) continue;
    oe_sort<KMAX, 0, KMAX>(blk);
#pragma unroll
    for (int s = 0; s < KMAX; ++s) list[s] = list[s] < blk[KMAX - 1 - s] ? list[s] : blk[KMAX - 1 - s];
    bitonic_sort(list);
  }
  uint64_t unused = 0;
  merge_round<KMAX, L, 1>(list, unused);
}

// The queries of a workgroup are kThreads / L consecutive (molecule, atom)
// pairs of the flattened batch, so no lane idles at the end of a molecule.
// The workgroup stages every molecule its queries touch, molecule m at
// m * stride (stride = N rounded up to 16 for N >= 64, so a block of 16
// consecutive candidates is one aligned 64-byte run per coordinate), plus
// L * KMAX zeroed entries after the last, which the unconditional reads of a
// final partial block reach.  code_stage_entries() is the host-side bound.
constexpr int kCodeStage = 1024;

__host__ __device__ constexpr int code_stride(int n) { return n >= 64 ? (n + 15) / 16 * 16 : n; }
__host__ __device__ constexpr int code_stage_entries(int n, int queries, int tail) {
  return (1 + (queries - 1 + n - 1) / n) * code_stride(n) + tail;
}

// Four waves per SIMD (at most 128 VGPRs; the spill this costs is in the
// rarely taken 64-bit recomputation) measured 12 % faster than three.
template <int KMAX, int L>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) knn_code_kernel(Params p) {
  __shared__ __align__(16) float stage_x[kCodeStage];
  __shared__ __align__(16) float stage_y[kCodeStage];
  __shared__ __align__(16) float stage_z[kCodeStage];
  __shared__ __align__(16) uint8_t stage_pad[kCodeStage];
  __shared__ uint32_t stage_bad[kCodeStage / 32 + 2];  // bit e: entry e is no valid atom

  constexpr int kQueries = kThreads / L;
  const int tid = threadIdx.x;
  const int sub = tid % L;
  const int N = p.N;  // <= kCodeAtoms (checked on the host)
  const int stride = code_stride(N);
  const long long total = (long long)p.B * N;
  const long long q0 = (long long)blockIdx.x * kQueries;
  const long long q = q0 + tid / L;
  const int b_first = int(q0 / N);
  const int b_last = int(min(total - 1, q0 + kQueries - 1) / N);
  const int staged = (b_last - b_first + 1) * stride;
  const float* x = p.coords + size_t(b_first) * N * 3;
  const uint8_t* pad = p.pad ? p.pad + size_t(b_first) * N : nullptr;
  // (wave-uniform trip count: the bad-entry bitmap is written by ballots)
  for (int e0 = 0; e0 < staged + L * KMAX; e0 += kThreads) {
    const int e = e0 + tid;
    const int m = e / stride;
    const int u = e - m * stride;
    const bool real = e < staged && u < N;
    const int a = m * N + u;
    const uint8_t padded = real ? (pad ? pad[a] : 0) : 1;
    if (e < kCodeStage) {
      stage_x[e] = real ? x[3 * a + 0] : 0.0f;
      stage_y[e] = real ? x[3 * a + 1] : 0.0f;
      stage_z[e] = real ? x[3 * a + 2] : 0.0f;
      stage_pad[e] = padded;
    }
    const unsigned long long bad = __ballot(padded != 0);
    if ((tid & 63) == 0 && e < kCodeStage) {
      stage_bad[e >> 5] = uint32_t(bad);
      stage_bad[(e >> 5) + 1] = uint32_t(bad >> 32);
    }
  }
  __syncthreads();
  const bool in_batch = q < total;
  const int b = in_batch ? int(q / N) : b_last;
  const int i = in_batch ? int(q - (long long)b * N) : N;
  const int base = (b - b_first) * stride;
  const float* sx = stage_x + base;
  const float* sy = stage_y + base;
  const float* sz = stage_z + base;
  const uint8_t* spad = stage_pad + base;
  const bool valid_i = in_batch && !spad[i];
  float xi = 0.0f, yi = 0.0f, zi = 0.0f;
  if (valid_i) {
    xi = sx[i];
    yi = sy[i];
    zi = sz[i];
  }
  // self is excluded by index; an invalid query takes i = -1 and a pad byte
  // test that every candidate fails
  const int self = p.exclude_self ? i : -1;
  const uint8_t live = valid_i ? 0 : 0xff;

  uint32_t list[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) list[s] = kEmpty32;
  uint32_t out_min = kEmpty32;
  // every lane runs the same number of blocks, so the wave stays converged;
  // the keys are computed without branches (reads past N stay inside the
  // staged region and are masked by u < N)
  for (int u0 = sub; u0 - sub < N; u0 += L * KMAX) {
    uint32_t blk[KMAX];
    bool below = false;
    if constexpr (L == 1) {
      // one exclusion bit per candidate of the block: staged padding and
      // gaps, columns past N, self, an invalid query; bit t set turns key t
      // into kEmpty32 (sign-extended bit OR-ed into the code)
      const int g = base + u0;
      uint32_t ex = __builtin_amdgcn_alignbit(stage_bad[(g >> 5) + 1], stage_bad[g >> 5], uint32_t(g & 31));
      const int rel_n = N - u0;
      if (rel_n < 32) ex |= ~0u << rel_n;
      const unsigned rel_i = unsigned(self - u0);
      ex |= rel_i < 32u ? 1u << rel_i : 0u;
      ex |= live ? ~0u : 0u;
#pragma unroll
      for (int t = 0; t < KMAX; ++t) {
        const int u = u0 + t;
        const float d2 = pair_d2(xi, yi, zi, sx[u], sy[u], sz[u]);
        const uint32_t code = ((__float_as_uint(d2) >> 7) << 8) | uint32_t(u);
        blk[t] = code | uint32_t(__builtin_amdgcn_sbfe(int(ex), t, 1));
        below |= blk[t] < list[KMAX - 1];
      }
    } else {
#pragma unroll
      for (int t = 0; t < KMAX; ++t) {
        const int u = u0 + L * t;
        const float d2 = pair_d2(xi, yi, zi, sx[u], sy[u], sz[u]);
        const uint32_t code = ((__float_as_uint(d2) >> 7) << 8) | uint32_t(u);
        const bool ok = ((spad[u] | live) == 0) & (u != self) & (u < N);
        blk[t] = ok ? code : kEmpty32;
        below |= blk[t] < list[KMAX - 1];
      }
    }
    if (!__any(below)) {
#pragma unroll
      for (int t = 0; t < KMAX; ++t) out_min = out_min < blk[t] ? out_min : blk[t];
      continue;
    }
    oe_sort<KMAX, 0, KMAX>(blk);
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      const uint32_t a = list[s], c = blk[KMAX - 1 - s];
      list[s] = a < c ? a : c;
      const uint32_t hi = a < c ? c : a;
      out_min = out_min < hi ? out_min : hi;
    }
    bitonic_sort(list);
  }
  merge_round<KMAX, L, 1, true>(list, out_min);

  if (!in_batch) return;  // whole query groups leave together
  const int k = p.K;
  uint32_t kth = kEmpty32, next = out_min;
  bool shared_code = false;  // two kept keys with one d2 code: their order needs the exact d2
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s == k - 1) kth = list[s];
    if (s == k) next = list[s];
    if (s > 0 && s < k) shared_code |= list[s] != kEmpty32 && (list[s] >> 8) == (list[s - 1] >> 8);
  }
  const bool ambiguous = kth != kEmpty32 && next != kEmpty32 && (kth >> 8) == (next >> 8);

  uint64_t fin[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    const uint32_t key = list[s];
    const int j = int(key & 0xffu);
    fin[s] = key == kEmpty32
                 ? kEmpty
                 : (static_cast<uint64_t>(__float_as_uint(pair_d2(xi, yi, zi, sx[j], sy[j], sz[j]))) << 32) | uint32_t(j);
  }
  if (__any(shared_code)) oe_sort<KMAX, 0, KMAX>(fin);
  if (__any(ambiguous)) {
    if (ambiguous) exact_scan<KMAX, L>(fin, sx, sy, sz, spad, N, i, sub, valid_i, p.exclude_self, xi, yi, zi);
  }

  int32_t* oi = p.idx + size_t(q) * p.K;
  float* od = p.dist ? p.dist + size_t(q) * p.K : nullptr;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s % L != sub || s >= k) continue;
    const uint64_t key = fin[s];
    const bool empty = key == kEmpty;
    oi[s] = empty ? -1 : static_cast<int32_t>(static_cast<uint32_t>(key));
    if (od) od[s] = empty ? INFINITY : sqrtf(__uint_as_float(static_cast<uint32_t>(key >> 32)));
  }
}

template <int KMAX, int L>
__global__ void __launch_bounds__(kThreads) knn_kernel(Params p) {
  __shared__ float sx[kTile], sy[kTile], sz[kTile];
  __shared__ uint8_t spad[kTile];

  constexpr int kQueries = kThreads / L;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int sub = tid % L;
  const int i = blockIdx.x * kQueries + tid / L;
  const int N = p.N;
  const float* x = p.coords + size_t(b) * N * 3;
  const uint8_t* pad = p.pad ? p.pad + size_t(b) * N : nullptr;
  const bool valid_i = i < N && !(pad && pad[i]);
  float xi = 0.0f, yi = 0.0f, zi = 0.0f;
  if (valid_i) {
    xi = x[3 * i + 0];
    yi = x[3 * i + 1];
    zi = x[3 * i + 2];
  }

  uint64_t list[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) list[s] = kEmpty;

  for (int t0 = 0; t0 < N; t0 += kTile) {
    const int n = min(kTile, N - t0);
    __syncthreads();
    for (int u = tid; u < n; u += kThreads) {
      sx[u] = x[3 * (t0 + u) + 0];
      sy[u] = x[3 * (t0 + u) + 1];
      sz[u] = x[3 * (t0 + u) + 2];
      spad[u] = pad ? pad[t0 + u] : 0;
    }
    __syncthreads();
    if (!valid_i) continue;
    for (int u = sub; u < n; u += L) {
      const int j = t0 + u;
      if (spad[u] || (p.exclude_self && j == i)) continue;
      const float dx = xi - sx[u];
      const float dy = yi - sy[u];
      const float dz = zi - sz[u];
      const float xx = dx * dx;
      const float yy = dy * dy;
      const float zz = dz * dz;
      const float s = xx + yy;
      const float d2 = s + zz;
      const uint64_t key = (static_cast<uint64_t>(__float_as_uint(d2)) << 32) | static_cast<uint32_t>(j);
      if (key < list[KMAX - 1]) insert(list, key);
    }
  }

  // butterfly merge of the L lane lists of a query
#pragma unroll
  for (int mask = 1; mask < L; mask <<= 1) {
#pragma unroll
    for (int s = 0; s < KMAX / 2; ++s) {
      const uint64_t other_hi = shfl_xor_u64(list[KMAX - 1 - s], mask);
      const uint64_t other_lo = shfl_xor_u64(list[s], mask);
      list[s] = list[s] < other_hi ? list[s] : other_hi;
      list[KMAX - 1 - s] = list[KMAX - 1 - s] < other_lo ? list[KMAX - 1 - s] : other_lo;
    }
    bitonic_sort(list);
  }

  if (i >= N) return;
  int32_t* oi = p.idx + (size_t(b) * N + i) * p.K;
  float* od = p.dist ? p.dist + (size_t(b) * N + i) * p.K : nullptr;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s % L != sub || s >= p.K) continue;
    const uint64_t key = list[s];
    const bool empty = key == kEmpty;
    oi[s] = empty ? -1 : static_cast<int32_t>(static_cast<uint32_t>(key));
    if (od) od[s] = empty ? INFINITY : sqrtf(__uint_as_float(static_cast<uint32_t>(key >> 32)));
  }
}

template <int KMAX, int L>
int launch(const Params& p, hipStream_t stream) {
  constexpr int kQueries = kThreads / L;
  const dim3 grid((p.N + kQueries - 1) / kQueries, p.B);
  if constexpr (KMAX <= 16) {
    // the code kernel for one lane per query (large batches); at a few lanes
    // per query its fixed per-query work (exact fix-up, flattened staging)
    // outweighs the cheaper comparators
    if constexpr (L == 1) {
      if (p.N <= kCodeAtoms && code_stage_entries(p.N, kQueries, KMAX) <= kCodeStage) {
        const long long blocks = ((long long)p.B * p.N + kQueries - 1) / kQueries;
        hipLaunchKernelGGL((knn_code_kernel<KMAX, 1>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream, p);
        MF_HIP_CHECK(hipGetLastError());
        return MF_OK;
      }
    }
    hipLaunchKernelGGL((knn_block_kernel<KMAX, L>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((knn_kernel<KMAX, L>), grid, dim3(kThreads), 0, stream, p);
  }
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

// Lanes per query: enough queries in flight to fill the GPU at small batch
// sizes, fewer lanes (less merging) when there are many queries.  The block
// kernel (k <= 16) goes down to one lane per query once the queries alone
// give every SIMD four waves.
template <int KMAX>
int dispatch_lanes(const Params& p, int num_cus, hipStream_t stream) {
  const long long queries = (long long)p.B * p.N;
  if constexpr (KMAX <= 16) {
    const long long lanes = (long long)num_cus * 4 * 4 * 64;
    if (queries >= lanes) return launch<KMAX, 1>(p, stream);
    if (queries * 2 >= lanes) return launch<KMAX, 2>(p, stream);
    if (queries * 4 >= lanes) return launch<KMAX, 4>(p, stream);
    if (queries * 8 >= lanes) return launch<KMAX, 8>(p, stream);
    return launch<KMAX, 16>(p, stream);
  } else {
    if (queries * 16 <= (long long)num_cus * 2048) return launch<KMAX, 16>(p, stream);
    if (queries * 8 <= (long long)num_cus * 4096) return launch<KMAX, 8>(p, stream);
    return launch<KMAX, 4>(p, stream);
  }
}

}  // namespace knn
}  // namespace mf

extern "C" int mf_knn(const mf_knn_args* a, void* stream) {
  using namespace mf;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn: args is NULL");
  if (!a->coords || !a->idx) return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn: coords and idx must be non-NULL");
  if (a->batch < 0 || a->atoms < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn: batch and atoms must be non-negative");
  if (a->k < 1 || a->k > 64) return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn: k must be in [1, 64]");
  if (a->batch > 65535) return fail(MF_ERR_UNSUPPORTED, "mf_knn: batch must be <= 65535");
  if (a->batch == 0 || a->atoms == 0) return MF_OK;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  knn::Params p{a->coords, a->pad_mask, a->idx, a->dist, a->batch, a->atoms, a->k, a->exclude_self != 0};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->k <= 8) return knn::dispatch_lanes<8>(p, dev.num_cus, s);
  if (a->k <= 16) return knn::dispatch_lanes<16>(p, dev.num_cus, s);
  if (a->k <= 32) return knn::dispatch_lanes<32>(p, dev.num_cus, s);
  return knn::launch<64, 4>(p, s);
}

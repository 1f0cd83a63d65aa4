// Cutoff (radius) neighbour bit masks, with the minimum image for periodic
// cells (mf_radius_mask), on gfx950.
//
// Pair distance of the reference's geometry adapters
// (src/matterformer/geometry/adapters.py): periodic d2 = min over the integer
// image offsets o in {-r..r}^3 (:141-149) of e^T G e, e = (f_i - f_j) + o,
// G = cell cell^T (:176-190); non-periodic d2 = |x_i - x_j|^2 (:98-99).  The
// fp32 evaluation order is fixed (this file is built with -ffp-contract=off):
//   t_c = (G[c][0]*e0 + G[c][1]*e1) + G[c][2]*e2,  d2 = (e0*t0 + e1*t1) + e2*t2
//   non-periodic: d2 = (dx*dx + dy*dy) + dz*dz
// and mask[i,j] = d2 <= cutoff*cutoff for valid i, j.
//
// Layout: one workgroup of four waves per T x T tile (T = max(block, 64));
// wave w owns T/4 rows of it.  Lane l owns column l of each 64-column chunk
// and keeps that atom's coordinates in registers; a row's coordinates are
// read from LDS at a wave-uniform address.  For one (row, chunk) the 64 lanes
// test their pairs and the wave's compare mask IS the row's two output words,
// which v_writelane parks in the lane that stores them.  The block mask
// entries of the tile are ORs of those masks, written by the workgroup that
// owns the tile, so no zero-fill pass and no atomics are needed.
//
// Image pruning (exact).  Only "does some image have d2 <= rc^2" matters.  If
// the computed d2 of image e is <= rc^2 then, with the rounding of the fp32
// quadratic form bounded by 5u |e|^T|G||e| <= 5u k' e^T G e
// (k' = maxrowsum|G| * trace(G^-1), u = 2^-24), e^T G e <= rc^2 / (1 - delta)
// and therefore e_c^2 <= rc^2 (G^-1)_cc / (1 - delta) for each component c
// (the largest e_c on that ellipsoid).  So an image with |e_c| above
// bound_c = sqrt(rc^2 (G^-1)_cc / (1 - delta)) for some c cannot be inside the
// cutoff, and skipping it cannot change the mask: the remaining images are
// evaluated with the same fp32 operations as the full search.  delta = 1e-3
// is used when 5u k' < 1e-4; otherwise (near-singular or very skewed cells)
// every image is evaluated.  For cells of MOF size (15-30 A, angles 80-100
// degrees) and a 6 A cutoff bound_c < 0.5, so at most one image survives.
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace radius {

struct Params {
  const float* coords;
  const float* gram;
  const uint8_t* pad;
  uint32_t* bits;
  uint8_t* block_mask;
  float rc2;
  int B, N, W, NB, NT;  // NB = ceil(N / block), NT = ceil(N / T)
};

// Per-cell pruning bounds (double precision; every lane computes the same
// values).
__device__ __forceinline__ void cell_bounds(const float* G, float rc2, float* bound) {
  double g[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) g[t] = G[t];
  const double c00 = g[4] * g[8] - g[5] * g[7];
  const double c11 = g[0] * g[8] - g[2] * g[6];
  const double c22 = g[0] * g[4] - g[1] * g[3];
  const double det = g[0] * c00 - g[1] * (g[3] * g[8] - g[5] * g[6]) + g[2] * (g[3] * g[7] - g[4] * g[6]);
  bool ok = det > 0.0 && std::isfinite(det);
  double inv[3] = {0, 0, 0};
  if (ok) {
    inv[0] = c00 / det;
    inv[1] = c11 / det;
    inv[2] = c22 / det;
    ok = inv[0] > 0 && inv[1] > 0 && inv[2] > 0;
  }
  if (ok) {
    double rowsum = 0.0;
    for (int r = 0; r < 3; ++r)
      rowsum = fmax(rowsum, fabs(g[3 * r]) + fabs(g[3 * r + 1]) + fabs(g[3 * r + 2]));
    const double kappa = rowsum * (inv[0] + inv[1] + inv[2]);
    ok = 5.0 * 0x1p-24 * kappa < 1e-4;
  }
  for (int c = 0; c < 3; ++c) {
    // rounded up to the next float so that the fp32 comparison stays conservative
    bound[c] = ok ? nextafterf(static_cast<float>(sqrt(double(rc2) * inv[c] / (1.0 - 1e-3))), INFINITY) : INFINITY;
  }
}

// True when every bound of cell_bounds is below 1/2, decided without a
// division or square root (det > 0): bound_c^2 = rc^2 cof_cc / (det (1 - delta))
// < 1/4, and the conditioning test 5u maxrowsum |G| trace(cof) < 1e-4 det.  A
// relative margin of 1e-9 covers the rounding of these double products, so a
// true result implies bounds below 1/2; a false one only selects the general
// search, which is exact for any cell.
__device__ __forceinline__ bool cell_is_nearest(const float* G, float rc2) {
  double g[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) g[t] = G[t];
  const double c00 = g[4] * g[8] - g[5] * g[7];
  const double c11 = g[0] * g[8] - g[2] * g[6];
  const double c22 = g[0] * g[4] - g[1] * g[3];
  const double det = g[0] * c00 - g[1] * (g[3] * g[8] - g[5] * g[6]) + g[2] * (g[3] * g[7] - g[4] * g[6]);
  double rowsum = 0.0;
#pragma unroll
  for (int r = 0; r < 3; ++r) rowsum = fmax(rowsum, fabs(g[3 * r]) + fabs(g[3 * r + 1]) + fabs(g[3 * r + 2]));
  const double lim = 0.25 * (1.0 - 1e-3) * (1.0 - 1e-9) * det;
  const double r2 = double(rc2);
  return det > 0.0 && det < INFINITY && c00 > 0.0 && c11 > 0.0 && c22 > 0.0 &&
         5.0 * 0x1p-24 * rowsum * (c00 + c11 + c22) < 1e-4 * (1.0 - 1e-9) * det &&
         r2 * c00 < lim && r2 * c11 < lim && r2 * c22 < lim;
}

template <int R>
__device__ __forceinline__ bool periodic_hit(float fi0, float fi1, float fi2, float fj0, float fj1, float fj2,
                                             const float* G, const float* bound, float rc2) {
  constexpr int NO = 2 * R + 1;
  const float d0 = fi0 - fj0;
  const float d1 = fi1 - fj1;
  const float d2v = fi2 - fj2;
  float e0[NO], e1[NO], e2[NO];
  bool a0[NO], a1[NO], a2[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) {
    const float off = static_cast<float>(o - R);
    e0[o] = d0 + off;
    e1[o] = d1 + off;
    e2[o] = d2v + off;
    a0[o] = fabsf(e0[o]) <= bound[0];
    a1[o] = fabsf(e1[o]) <= bound[1];
    a2[o] = fabsf(e2[o]) <= bound[2];
  }
  bool hit = false;
#pragma unroll
  for (int o0 = 0; o0 < NO; ++o0) {
    if (!a0[o0]) continue;
#pragma unroll
    for (int o1 = 0; o1 < NO; ++o1) {
      if (!a1[o1]) continue;
      // (G[c][0]*e0 + G[c][1]*e1) is shared by the images that differ in o2
      float s01[3];
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        const float p0 = G[3 * c + 0] * e0[o0];
        const float p1 = G[3 * c + 1] * e1[o1];
        s01[c] = p0 + p1;
      }
#pragma unroll
      for (int o2 = 0; o2 < NO; ++o2) {
        if (!a2[o2]) continue;
        float t[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const float p2 = G[3 * c + 2] * e2[o2];
          t[c] = s01[c] + p2;
        }
        const float q0 = e0[o0] * t[0];
        const float q1 = e1[o1] * t[1];
        const float q2 = e2[o2] * t[2];
        const float s = q0 + q1;
        const float dd = s + q2;
        hit = hit || dd <= rc2;
      }
    }
  }
  return hit;
}

// All image bounds below 1/2: of the offsets o_c, only the one nearest to
// -d_c can leave |d_c + o_c| <= bound_c, so at most one image can be inside
// the cutoff: o = -rint(d), clamped to the searched range {-R..R} (the
// coordinates need not lie in [0, 1), and an offset outside the range is not
// an image the search considers; after the clamp every |e_c| of the other
// images still exceeds 1/2).  It is evaluated with the same operations (and
// order) as the full search, so the decision is identical.  No bound test is
// needed on it: a computed d2 <= rc^2 implies |e_c| <= bound_c.
template <int R>
__device__ __forceinline__ bool nearest_image_hit(float fi0, float fi1, float fi2, float fj0, float fj1, float fj2,
                                                  const float* G, float rc2) {
  constexpr float fr = static_cast<float>(R);
  const float d0 = fi0 - fj0;
  const float d1 = fi1 - fj1;
  const float d2v = fi2 - fj2;
  const float e0 = d0 + fminf(fmaxf(-rintf(d0), -fr), fr);
  const float e1 = d1 + fminf(fmaxf(-rintf(d1), -fr), fr);
  const float e2 = d2v + fminf(fmaxf(-rintf(d2v), -fr), fr);
  float t[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float p0 = G[3 * c + 0] * e0;
    const float p1 = G[3 * c + 1] * e1;
    const float s01 = p0 + p1;
    const float p2 = G[3 * c + 2] * e2;
    t[c] = s01 + p2;
  }
  const float q0 = e0 * t[0];
  const float q1 = e1 * t[1];
  const float q2 = e2 * t[2];
  const float s = q0 + q1;
  return s + q2 <= rc2;
}

__device__ __forceinline__ bool plain_hit(float xi, float yi, float zi, float xj, float yj, float zj, float rc2) {
  const float dx = xi - xj;
  const float dy = yi - yj;
  const float dz = zi - zj;
  const float xx = dx * dx;
  const float yy = dy * dy;
  const float zz = dz * dz;
  const float s = xx + yy;
  return s + zz <= rc2;
}

// Parks the 64-bit compare mask of (row r, chunk c) in the lanes that store
// its two words: word e = 2 (r CH + c) + h of the wave lives in lane e % 64 of
// words[e / 64] (e is even, so both words land in the same register).
template <int NW>
__device__ __forceinline__ void park(uint32_t (&words)[NW], uint64_t m, int e, int lane) {
#pragma unroll
  for (int n = 0; n < NW; ++n) {
    if ((e >> 6) == n) {
      words[n] = lane == (e & 63) ? static_cast<uint32_t>(m) : words[n];
      words[n] = lane == (e & 63) + 1 ? static_cast<uint32_t>(m >> 32) : words[n];
    }
  }
}

// Coordinate k of the wave's rows: lane k % 64 of ci[k / 64] (k wave-uniform).
template <int NI>
__device__ __forceinline__ float row_coord(const float (&ci)[NI], int k) {
  float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ci[0]), k & 63));
#pragma unroll
  for (int n = 1; n < NI; ++n) {
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ci[n]), k & 63));
    v = (k >> 6) == n ? w : v;
  }
  return v;
}

// MODE: 0 non-periodic, 1 periodic r=1, 2 periodic r=2
template <int BLOCK, int MODE>
__global__ void __launch_bounds__(256) radius_mask_kernel(Params p) {
  constexpr int T = BLOCK < 64 ? 64 : BLOCK;  // tile edge
  constexpr int CH = T / 64;                  // 64-column chunks per tile row
  constexpr int RPW = T / 4;                  // rows per wave
  constexpr int WPW = RPW * 2 * CH;           // output words per wave
  constexpr int NW = (WPW + 63) / 64;
  constexpr int NI = (3 * RPW + 63) / 64;     // registers of row coordinates
  constexpr int TW = T / 32;                  // words per tile row
  __shared__ uint32_t s_tr[4][CH][64];
  __shared__ uint32_t s_any[4];

  // Tile (ti, tj), ti <= tj, of the upper triangle; the mask is symmetric
  // (d2(i, j) and d2(j, i) are the same fp32 value: e negates exactly and the
  // image set is symmetric), so the workgroup also writes tile (tj, ti).
  // Row ti of the triangle starts at index ti NT - ti (ti - 1) / 2.
  // XCD-aware order: consecutive workgroups land on different XCDs (linear
  // id % 8), so the logical unit is remapped to give each XCD whole cells;
  // a cell's row pieces (its tiles and their mirrors write 8- and 4-byte
  // pieces of shared 64-byte rows) then merge in one L2 before they reach
  // HBM.
  const long long tiles = (long long)p.NT * (p.NT + 1) / 2;
  const long long grid = (long long)gridDim.x;
  const long long unit = (blockIdx.x & 7) * (grid >> 3) + (blockIdx.x >> 3);
  if (unit >= tiles * p.B) return;  // grid padding (whole workgroup)
  const int b = int(unit / tiles);
  const long long nt = p.NT, t = unit - (long long)b * tiles;
  auto row_start = [nt](long long r) { return r * nt - r * (r - 1) / 2; };
  const double q = double(2 * nt + 1);
  long long r0 = static_cast<long long>((q - sqrt(q * q - 8.0 * double(t))) * 0.5);
  r0 = r0 < 0 ? 0 : (r0 > nt - 1 ? nt - 1 : r0);
  while (r0 > 0 && row_start(r0) > t) --r0;
  while (r0 + 1 < nt && row_start(r0 + 1) <= t) ++r0;
  const int ti = static_cast<int>(r0);
  const int tj = static_cast<int>(ti + (t - row_start(r0)));
  const bool mirror = ti != tj;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = p.N;
  const float* x = p.coords + size_t(b) * N * 3;
  const uint8_t* pad = p.pad ? p.pad + size_t(b) * N : nullptr;
  const int row0 = ti * T + wave * RPW;

  float xj[CH][3];
  uint64_t vj[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = tj * T + c * 64 + lane;
    const bool in = j < N;
    xj[c][0] = in ? x[3 * j + 0] : 0.0f;
    xj[c][1] = in ? x[3 * j + 1] : 0.0f;
    xj[c][2] = in ? x[3 * j + 2] : 0.0f;
    vj[c] = __ballot(in && !(pad && pad[j]));
  }
  float ci[NI];
#pragma unroll
  for (int n = 0; n < NI; ++n) {
    const int e = n * 64 + lane;
    ci[n] = e < 3 * RPW && 3 * row0 + e < 3 * N ? x[3 * row0 + e] : 0.0f;
  }
  const uint64_t vi = __ballot(lane < RPW && row0 + lane < N && !(pad && pad[row0 + lane]));

  float G[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0}, bound[3] = {INFINITY, INFINITY, INFINITY};
  bool nearest = false;
  if constexpr (MODE != 0) {
    const float g = lane < 9 ? p.gram[size_t(b) * 9 + lane] : 0.0f;
#pragma unroll
    for (int k = 0; k < 9; ++k) G[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), k));
    nearest = cell_is_nearest(G, p.rc2);  // per cell
    if (!nearest) cell_bounds(G, p.rc2, bound);
  }

  uint32_t words[NW], tw[CH];
#pragma unroll
  for (int n = 0; n < NW; ++n) words[n] = 0u;
#pragma unroll
  for (int c = 0; c < CH; ++c) tw[c] = 0u;
  uint32_t any_lo = 0u, any_hi = 0u;
  // Row r of the wave: the 64 lanes test their pairs; the compare mask is the
  // row's words, and each lane's own bit goes to its transposed word.
  auto row_masks = [&](int r, auto hit_fn) {
    const float fi0 = row_coord(ci, 3 * r), fi1 = row_coord(ci, 3 * r + 1), fi2 = row_coord(ci, 3 * r + 2);
    const bool row_ok = (vi >> r) & 1u;
    const uint32_t tbit = 1u << ((wave * RPW + r) & 31);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool h = hit_fn(fi0, fi1, fi2, xj[c][0], xj[c][1], xj[c][2]) & row_ok;
      const uint64_t m = __ballot(h) & vj[c];
      park(words, m, 2 * (r * CH + c), lane);
      any_lo |= static_cast<uint32_t>(m);
      any_hi |= static_cast<uint32_t>(m >> 32);
      tw[c] = h ? tw[c] | tbit : tw[c];
    }
  };
  const float rc2 = p.rc2;
  if constexpr (MODE == 0) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      row_masks(r, [&](float a0, float a1, float a2, float b0, float b1, float b2) {
        return plain_hit(a0, a1, a2, b0, b1, b2, rc2);
      });
  } else if (nearest) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      row_masks(r, [&](float a0, float a1, float a2, float b0, float b1, float b2) {
        return nearest_image_hit<MODE>(a0, a1, a2, b0, b1, b2, G, rc2);
      });
  } else {
#pragma unroll 1
    for (int r = 0; r < RPW; ++r)
      row_masks(r, [&](float a0, float a1, float a2, float b0, float b1, float b2) {
        return periodic_hit<MODE>(a0, a1, a2, b0, b1, b2, G, bound, rc2);
      });
  }

  // Tile (ti, tj): row row0 + r, word tj * TW + e % (2 CH).
#pragma unroll
  for (int n = 0; n < NW; ++n) {
    const int e = n * 64 + lane;
    const int r = e / (2 * CH), w = tj * TW + e % (2 * CH);
    if (e < WPW && row0 + r < N && w < p.W) p.bits[(size_t(b) * N + row0 + r) * p.W + w] = words[n];
  }
  if (mirror) {
#pragma unroll
    for (int c = 0; c < CH; ++c) s_tr[wave][c][lane] = ((vj[c] >> lane) & 1u) ? tw[c] : 0u;
  }
  if (lane == 0) s_any[wave] = (any_lo != 0u ? 1u : 0u) | (any_hi != 0u ? 2u : 0u);
  __syncthreads();

  // Tile (tj, ti): row tj T + 64 c + lane, word ti TW + k; word k gathers the
  // bits of tile rows 32k .. 32k+31, held by waves 32k / RPW .. (32k+31) / RPW.
  if (mirror) {
    for (int item = wave; item < TW * CH; item += 4) {
      const int k = item / CH, c = item - k * CH;
      uint32_t v = 0u;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        if (w * RPW < 32 * k + 32 && w * RPW + RPW > 32 * k) v |= s_tr[w][c][lane];
      const int row = tj * T + c * 64 + lane, col = ti * TW + k;
      if (row < N && col < p.W) p.bits[(size_t(b) * N + row) * p.W + col] = v;
    }
  }

  if (p.block_mask == nullptr || threadIdx.x >= 4) return;
  if constexpr (BLOCK == T) {
    if (threadIdx.x == 0) {
      const uint8_t any = (s_any[0] | s_any[1] | s_any[2] | s_any[3]) != 0u ? 1 : 0;
      p.block_mask[(size_t(b) * p.NB + ti) * p.NB + tj] = any;
      if (mirror) p.block_mask[(size_t(b) * p.NB + tj) * p.NB + ti] = any;
    }
  } else {
    // block 32: wave w's rows lie in row half w / 2 of the 64 x 64 tile;
    // the low and high mask words are the two column halves.
    const int hr = threadIdx.x >> 1, hc = threadIdx.x & 1;
    const int bi = 2 * ti + hr, bj = 2 * tj + hc;
    const uint8_t any = ((s_any[2 * hr] | s_any[2 * hr + 1]) >> hc) & 1u;
    if (bi < p.NB && bj < p.NB) {
      p.block_mask[(size_t(b) * p.NB + bi) * p.NB + bj] = any;
      if (mirror) p.block_mask[(size_t(b) * p.NB + bj) * p.NB + bi] = any;
    }
  }
}

template <int BLOCK, int MODE>
int launch(const Params& p, hipStream_t stream) {
  const long long units = (long long)p.NT * (p.NT + 1) / 2 * p.B;
  const dim3 grid(unsigned((units + 7) / 8 * 8));  // a multiple of 8 (one share per XCD)
  hipLaunchKernelGGL((radius_mask_kernel<BLOCK, MODE>), grid, dim3(256), 0, stream, p);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

template <int BLOCK>
int dispatch_mode(const Params& p, int mode, hipStream_t stream) {
  if (mode == 0) return launch<BLOCK, 0>(p, stream);
  if (mode == 1) return launch<BLOCK, 1>(p, stream);
  return launch<BLOCK, 2>(p, stream);
}

}  // namespace radius
}  // namespace mf

extern "C" int mf_radius_mask(const mf_radius_mask_args* a, void* stream) {
  using namespace mf;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_mask: args is NULL");
  if (!a->coords || !a->mask_bits)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_mask: coords and mask_bits must be non-NULL");
  if (a->batch < 0 || a->atoms < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_mask: batch and atoms must be non-negative");
  if (a->block != 32 && a->block != 64 && a->block != 128)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_mask: block must be 32, 64 or 128");
  if (a->gram && a->pbc_radius != 1 && a->pbc_radius != 2)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_mask: pbc_radius must be 1 or 2");
  if (!(a->cutoff > 0.0f) || !std::isfinite(a->cutoff))
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_radius_mask: cutoff must be positive and finite");
  if (a->batch == 0 || a->atoms == 0) return MF_OK;
  const long long nb = (a->atoms + a->block - 1) / a->block;
  const int tile = a->block < 64 ? 64 : a->block;
  const long long nt = (a->atoms + tile - 1) / tile;
  if (a->batch > 65535 || nt * (nt + 1) / 2 * a->batch > 0x7ffffff0LL)
    return fail(MF_ERR_UNSUPPORTED, "mf_radius_mask: batch or atom count too large");
  radius::Params p{a->coords, a->gram, a->pad_mask, a->mask_bits, a->block_mask,
                   a->cutoff * a->cutoff, a->batch, a->atoms, (a->atoms + 31) / 32, static_cast<int>(nb),
                   static_cast<int>(nt)};
  const int mode = a->gram ? a->pbc_radius : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->block == 32) return radius::dispatch_mode<32>(p, mode, s);
  if (a->block == 64) return radius::dispatch_mode<64>(p, mode, s);
  return radius::dispatch_mode<128>(p, mode, s);
}

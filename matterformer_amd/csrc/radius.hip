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
// Layout: one workgroup per (cell, i block, j block) of a block x block tile;
// thread (row r, word w) evaluates the 32 pairs of one output word.  The j
// block's coordinates sit in LDS.  The block mask entry of the tile is the OR
// of the workgroup's words, written by one thread, so no zero-fill pass and no
// atomics are needed.
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
  int B, N, W, NB;
};

// Per-cell pruning bounds (double precision, once per workgroup).
__device__ void cell_bounds(const float* G, float rc2, float* bound) {
  double g[9];
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
// the cutoff: o = -rint(d).  It is evaluated with the same operations (and
// order) as the full search, so the decision is identical.
__device__ __forceinline__ bool nearest_image_hit(float fi0, float fi1, float fi2, float fj0, float fj1, float fj2,
                                                  const float* G, const float* bound, float rc2) {
  const float d0 = fi0 - fj0;
  const float d1 = fi1 - fj1;
  const float d2v = fi2 - fj2;
  const float e0 = d0 + (-rintf(d0));
  const float e1 = d1 + (-rintf(d1));
  const float e2 = d2v + (-rintf(d2v));
  if (fabsf(e0) > bound[0] || fabsf(e1) > bound[1] || fabsf(e2) > bound[2]) return false;
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

// MODE: 0 non-periodic, 1 periodic r=1, 2 periodic r=2
template <int BLOCK, int MODE>
__global__ void __launch_bounds__(BLOCK * (BLOCK / 32)) radius_mask_kernel(Params p) {
  constexpr int WPB = BLOCK / 32;  // words per block row
  __shared__ float sj[3][BLOCK];
  __shared__ uint8_t spj[BLOCK];
  __shared__ float sG[9];
  __shared__ float sbound[3];

  const int b = blockIdx.y;
  const int ib = blockIdx.x / p.NB, jb = blockIdx.x % p.NB;
  const int tid = threadIdx.x;
  const int r = tid / WPB, ww = tid % WPB;
  const int N = p.N;
  const float* x = p.coords + size_t(b) * N * 3;
  const uint8_t* pad = p.pad ? p.pad + size_t(b) * N : nullptr;

  const int j0 = jb * BLOCK;
  for (int u = tid; u < BLOCK; u += BLOCK * WPB) {
    const int j = j0 + u;
    const bool in = j < N;
    sj[0][u] = in ? x[3 * j + 0] : 0.0f;
    sj[1][u] = in ? x[3 * j + 1] : 0.0f;
    sj[2][u] = in ? x[3 * j + 2] : 0.0f;
    spj[u] = (!in || (pad && pad[j])) ? 1 : 0;
  }
  if constexpr (MODE != 0) {
    if (tid < 9) sG[tid] = p.gram[size_t(b) * 9 + tid];
    if (tid == 0) cell_bounds(p.gram + size_t(b) * 9, p.rc2, sbound);
  }
  __syncthreads();

  const int i = ib * BLOCK + r;
  const bool valid_i = i < N && !(pad && pad[i]);
  uint32_t word = 0;
  if (valid_i) {
    const float xi = x[3 * i + 0], yi = x[3 * i + 1], zi = x[3 * i + 2];
    float G[9], bound[3];
    if constexpr (MODE != 0) {
#pragma unroll
      for (int t = 0; t < 9; ++t) G[t] = sG[t];
#pragma unroll
      for (int c = 0; c < 3; ++c) bound[c] = sbound[c];
    }
    bool nearest = false;
    if constexpr (MODE != 0) nearest = bound[0] < 0.5f && bound[1] < 0.5f && bound[2] < 0.5f;  // per cell
    if (nearest) {
      for (int t = 0; t < 32; ++t) {
        const int u = ww * 32 + t;
        if (!spj[u] && nearest_image_hit(xi, yi, zi, sj[0][u], sj[1][u], sj[2][u], G, bound, p.rc2))
          word |= 1u << t;
      }
    } else {
      for (int t = 0; t < 32; ++t) {
        const int u = ww * 32 + t;
        if (spj[u]) continue;
        bool hit;
        if constexpr (MODE == 0)
          hit = plain_hit(xi, yi, zi, sj[0][u], sj[1][u], sj[2][u], p.rc2);
        else
          hit = periodic_hit<MODE>(xi, yi, zi, sj[0][u], sj[1][u], sj[2][u], G, bound, p.rc2);
        if (hit) word |= 1u << t;
      }
    }
  }
  const int w = jb * WPB + ww;
  if (i < N && w < p.W) p.bits[(size_t(b) * N + i) * p.W + w] = word;
  const int any = __syncthreads_or(word != 0);
  if (p.block_mask && tid == 0) p.block_mask[(size_t(b) * p.NB + ib) * p.NB + jb] = any ? 1 : 0;
}

template <int BLOCK, int MODE>
int launch(const Params& p, hipStream_t stream) {
  const dim3 grid(p.NB * p.NB, p.B);
  hipLaunchKernelGGL((radius_mask_kernel<BLOCK, MODE>), grid, dim3(BLOCK * (BLOCK / 32)), 0, stream, p);
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
  if (a->batch > 65535 || nb * nb > 0x7fffffffLL)
    return fail(MF_ERR_UNSUPPORTED, "mf_radius_mask: batch or atom count too large");
  radius::Params p{a->coords, a->gram, a->pad_mask, a->mask_bits, a->block_mask,
                   a->cutoff * a->cutoff, a->batch, a->atoms, (a->atoms + 31) / 32, static_cast<int>(nb)};
  const int mode = a->gram ? a->pbc_radius : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->block == 32) return radius::dispatch_mode<32>(p, mode, s);
  if (a->block == 64) return radius::dispatch_mode<64>(p, mode, s);
  return radius::dispatch_mode<128>(p, mode, s);
}

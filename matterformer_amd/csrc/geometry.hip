// Pairwise geometry features in one pass (mf_geometry_features) on gfx950.
//
// The reference's adapters (src/matterformer/geometry/adapters.py) build
//   non-periodic (:83-125): delta = x_i - x_j, d2 = |delta|^2, d = sqrt(d2),
//                           d_norm = d / rms_radius
//   periodic (:151-212):    the 27 (or 125) image deltas (f_i - f_j) + o of
//                           every pair as a [B, N, N, 27, 3] tensor, their
//                           d2 = e^T G e, the argmin image, its delta and d2,
//                           d = sqrt(d2), d_norm = d / cell_scale
// and zero every output outside the valid-pair mask.  Here one wave takes
// one (molecule, row i, 64-column chunk): lane j evaluates the images in
// registers, keeps the first minimum in the reference's offset order
// (itertools.product over {-R..R}^3, last offset fastest), and writes the
// pair's outputs (coalesced across lanes); nothing per image reaches memory.
// The same pass can emit the cutoff mask of mf_radius_mask (d2 <= cutoff^2
// on valid pairs) as bits: the minimum over the images is below the cutoff
// iff some image is, and each image's d2 is evaluated with the operations of
// radius.hip in the same order, so the bits are identical.
//
// Arithmetic (every operation rounded; this file is built without FMA
// contraction): e_c = (f_ic - f_jc) + o_c;
//   t_c = (G[c][0] e_0 + G[c][1] e_1) + G[c][2] e_2;
//   d2  = (e_0 t_0 + e_1 t_1) + e_2 t_2;
// non-periodic d2 = (dx dx + dy dy) + dz dz, the order of the reference's
// square().sum(-1); sqrt and division correctly rounded.
#include <algorithm>
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace geom {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;

struct Params {
  const float* coords;
  const float* gram;
  const float* scale;
  const uint8_t* pad;
  uint8_t* pmask;
  float* delta;
  float* d2;
  float* dist;
  float* dnorm;
  uint32_t* bits;
  float rc2;
  int B, N, W, chunks;
};

template <int R>
__device__ __forceinline__ float min_image(float d0, float d1, float d2v, const float* G, float& e0o, float& e1o,
                                           float& e2o) {
  float best = INFINITY;
  e0o = d0;
  e1o = d1;
  e2o = d2v;
#pragma unroll
  for (int o0 = -R; o0 <= R; ++o0) {
    const float e0 = d0 + static_cast<float>(o0);
#pragma unroll
    for (int o1 = -R; o1 <= R; ++o1) {
      const float e1 = d1 + static_cast<float>(o1);
      float s01[3];
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        const float p0 = G[3 * c + 0] * e0;
        const float p1 = G[3 * c + 1] * e1;
        s01[c] = p0 + p1;
      }
#pragma unroll
      for (int o2 = -R; o2 <= R; ++o2) {
        const float e2 = d2v + static_cast<float>(o2);
        float t[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const float p2 = G[3 * c + 2] * e2;
          t[c] = s01[c] + p2;
        }
        const float q0 = e0 * t[0];
        const float q1 = e1 * t[1];
        const float q2 = e2 * t[2];
        const float s = q0 + q1;
        const float dd = s + q2;
        if (dd < best) {  // strict: the first minimum in offset order, as argmin
          best = dd;
          e0o = e0;
          e1o = e1;
          e2o = e2;
        }
      }
    }
  }
  return best;
}

// The non-periodic adapter's radius (adapters.py:116-118): one workgroup per
// molecule, sqrt(max(sum over valid atoms of |x|^2 / max(count, 1), 1e-8)),
// at least 1e-8.  |x|^2 = (x x + y y) + z z as square().sum(-1) rounds it.
__global__ void __launch_bounds__(kThreads) rms_kernel(const float* coords, const uint8_t* pad, float* scale, int N) {
  __shared__ float s_sum[kWavesPerBlock];
  __shared__ int s_cnt[kWavesPerBlock];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float sum = 0.0f;
  int cnt = 0;
  for (int a = tid; a < N; a += kThreads) {
    const size_t r = size_t(b) * N + a;
    if (pad != nullptr && pad[r] != 0) continue;
    const float x = coords[3 * r + 0], y = coords[3 * r + 1], z = coords[3 * r + 2];
    const float xx = x * x;
    const float yy = y * y;
    const float zz = z * z;
    const float s2 = xx + yy;
    sum += s2 + zz;
    ++cnt;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    sum += __shfl_xor(sum, off, 64);
    cnt += __shfl_xor(cnt, off, 64);
  }
  if (lane == 0) {
    s_sum[wave] = sum;
    s_cnt[wave] = cnt;
  }
  __syncthreads();
  if (tid == 0) {
    float t = 0.0f;
    int c = 0;
    for (int w = 0; w < kWavesPerBlock; ++w) {
      t += s_sum[w];
      c += s_cnt[w];
    }
    const float mean = t / float(c > 0 ? c : 1);
    scale[b] = fmaxf(sqrtf(fmaxf(mean, 1e-8f)), 1e-8f);
  }
}

template <int R>  // R = 0: non-periodic
__global__ void __launch_bounds__(kThreads) features_kernel(Params p) {
  const int lane = threadIdx.x & 63;
  const long long units = (long long)p.B * p.N * p.chunks;
  for (long long u = (long long)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6); u < units;
       u += (long long)gridDim.x * kWavesPerBlock) {
    const int chunk = int(u % p.chunks);
    const long long row = u / p.chunks;  // b * N + i
    const int i = int(row % p.N);
    const int b = int(row / p.N);
    const int j = chunk * 64 + lane;
    const bool in_row = j < p.N;
    const bool vi = p.pad == nullptr || p.pad[row] == 0;
    const bool vj = in_row && (p.pad == nullptr || p.pad[(long long)b * p.N + j] == 0);
    const bool ok = vi && vj;
    const float* ci = p.coords + row * 3;
    const float* cj = p.coords + ((long long)b * p.N + (in_row ? j : 0)) * 3;
    const float d0 = ci[0] - cj[0];
    const float d1 = ci[1] - cj[1];
    const float d2v = ci[2] - cj[2];
    float e0 = d0, e1 = d1, e2 = d2v, dd;
    if constexpr (R == 0) {
      const float xx = d0 * d0;
      const float yy = d1 * d1;
      const float zz = d2v * d2v;
      const float s = xx + yy;
      dd = s + zz;
    } else {
      float G[9];
#pragma unroll
      for (int c = 0; c < 9; ++c) G[c] = p.gram[(long long)b * 9 + c];
      dd = min_image<R>(d0, d1, d2v, G, e0, e1, e2);
    }
    dd = fmaxf(dd, 0.0f);
    if (in_row) {
      const long long o = row * p.N + j;
      if (p.delta) {
        p.delta[3 * o + 0] = ok ? e0 : 0.0f;
        p.delta[3 * o + 1] = ok ? e1 : 0.0f;
        p.delta[3 * o + 2] = ok ? e2 : 0.0f;
      }
      const float d = sqrtf(dd);
      if (p.d2) p.d2[o] = ok ? dd : 0.0f;
      if (p.dist) p.dist[o] = ok ? d : 0.0f;
      if (p.dnorm) p.dnorm[o] = ok ? d / p.scale[b] : 0.0f;
      if (p.pmask) p.pmask[o] = ok ? 1 : 0;
    }
    if (p.bits) {
      const unsigned long long m = __ballot(ok && dd <= p.rc2);
      const int w = 2 * chunk + (lane >> 5);
      if ((lane & 31) == 0 && w < p.W) p.bits[row * p.W + w] = uint32_t(lane ? m >> 32 : m);
    }
  }
}

// min(max(x, lo), hi) that keeps a NaN, as torch.clamp does
__device__ __forceinline__ float clampf(float x, float lo, float hi) { return x != x ? x : fminf(fmaxf(x, lo), hi); }

// The lattice terms of one cell per thread (lattice.py:12-131; adapters.py:173-174,192), each operation in
// the order the torch formulation applies it (this file is built without FMA contraction).
__global__ void __launch_bounds__(kThreads) lattice_kernel(const float* lat, int B, int repr, float* gram, float* y1,
                                                           float* cell_scale) {
  const int b = blockIdx.x * kThreads + threadIdx.x;
  if (b >= B) return;
  float l[6];
#pragma unroll
  for (int e = 0; e < 6; ++e) l[e] = lat[size_t(b) * 6 + e];
  float c[3][3] = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
  if (repr == MF_LATTICE_Y1) {
    const float l0 = expf(clampf(l[0], -5.0f, 5.0f));
    const float l1 = expf(clampf(l[1], -5.0f, 5.0f));
    const float l2 = expf(clampf(l[2], -5.0f, 5.0f));
    const float ca = clampf(l[3], -0.9999f, 0.9999f);
    const float cb = clampf(l[4], -0.9999f, 0.9999f);
    const float cgm = clampf(l[5], -0.9999f, 0.9999f);
    const float sg = sqrtf(fmaxf(1.0f - cgm * cgm, 1e-8f));
    c[0][0] = l0;
    c[1][0] = l1 * cgm;
    c[1][1] = l1 * sg;
    c[2][0] = l2 * cb;
    c[2][1] = (l2 * (ca - cb * cgm)) / sg;
    const float r = sqrtf((l2 * l2 - c[2][0] * c[2][0]) - c[2][1] * c[2][1]);
    c[2][2] = r != r ? r : fmaxf(r, 1e-8f);  // clamp_min keeps a NaN
  } else {
    c[0][0] = expf(clampf(l[0], -5.0f, 5.0f));
    c[1][1] = expf(clampf(l[2], -5.0f, 5.0f));
    c[2][2] = expf(clampf(l[5], -5.0f, 5.0f));
    c[1][0] = clampf(l[1], -10.0f, 10.0f);
    c[2][0] = clampf(l[3], -10.0f, 10.0f);
    c[2][1] = clampf(l[4], -10.0f, 10.0f);
  }
  float g[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const float v = (c[i][0] * c[j][0] + c[i][1] * c[j][1]) + c[i][2] * c[j][2];
      g[i][j] = isfinite(v) ? v : 0.0f;
    }
  if (gram) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) gram[size_t(b) * 9 + 3 * i + j] = g[i][j];
  }
  float y[6];
  if (repr == MF_LATTICE_Y1) {
#pragma unroll
    for (int e = 0; e < 3; ++e) y[e] = clampf(l[e], -5.0f, 5.0f);
#pragma unroll
    for (int e = 3; e < 6; ++e) y[e] = clampf(l[e], -0.9999f, 0.9999f);
  } else {  // gram_to_y1
    float len[3];
#pragma unroll
    for (int e = 0; e < 3; ++e) len[e] = sqrtf(fmaxf(g[e][e], 1e-8f));
    const float da = fmaxf(len[1] * len[2], 1e-8f), db = fmaxf(len[0] * len[2], 1e-8f),
                dg = fmaxf(len[0] * len[1], 1e-8f);
#pragma unroll
    for (int e = 0; e < 3; ++e) y[e] = logf(fmaxf(len[e], 1e-8f));
    y[3] = clampf(g[1][2] / da, -0.9999f, 0.9999f);
    y[4] = clampf(g[0][2] / db, -0.9999f, 0.9999f);
    y[5] = clampf(g[0][1] / dg, -0.9999f, 0.9999f);
  }
  if (y1) {
#pragma unroll
    for (int e = 0; e < 6; ++e) y1[size_t(b) * 6 + e] = y[e];
  }
  if (cell_scale) cell_scale[b] = fmaxf(((expf(y[0]) + expf(y[1])) + expf(y[2])) / 3.0f, 1e-8f);
}

}  // namespace geom
}  // namespace mf

extern "C" int mf_lattice_terms(const float* lattice, int32_t batch, int32_t lattice_repr, float* gram, float* y1,
                                float* cell_scale, void* stream) {
  using namespace mf;
  using namespace mf::geom;
  if (batch < 0) return fail(MF_ERR_INVALID_ARGUMENT, "mf_lattice_terms: batch must be non-negative");
  if (lattice_repr != MF_LATTICE_Y1 && lattice_repr != MF_LATTICE_LTRI)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_lattice_terms: unknown lattice_repr");
  if (batch == 0) return MF_OK;
  if (!lattice) return fail(MF_ERR_INVALID_ARGUMENT, "mf_lattice_terms: lattice must be non-NULL");
  hipLaunchKernelGGL(lattice_kernel, dim3(unsigned((batch + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), lattice, int(batch), int(lattice_repr), gram, y1, cell_scale);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

extern "C" int mf_geometry_features(const mf_geometry_args* a, void* stream) {
  using namespace mf;
  using namespace mf::geom;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: args is NULL");
  if (!a->coords) return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: coords must be non-NULL");
  if (a->batch < 0 || a->atoms < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: batch and atoms must be non-negative");
  if (a->pair_dist_norm && !a->scale)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: pair_dist_norm needs scale");
  if (a->scale_mode != MF_SCALE_GIVEN && a->scale_mode != MF_SCALE_RMS)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: unknown scale_mode");
  if (a->scale_mode == MF_SCALE_RMS && (!a->scale || a->gram))
    return fail(MF_ERR_INVALID_ARGUMENT,
                "mf_geometry_features: MF_SCALE_RMS needs a scale buffer and no gram (non-periodic)");
  if (a->mask_bits && !(a->cutoff > 0.0f))
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: mask_bits needs a positive cutoff");
  if (a->gram && a->pbc_radius != 1 && a->pbc_radius != 2)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_geometry_features: pbc_radius must be 1 or 2");
  if (a->batch == 0 || a->atoms == 0) return MF_OK;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  Params p{};
  p.coords = a->coords; p.gram = a->gram; p.scale = a->scale; p.pad = a->pad_mask; p.pmask = a->pair_mask;
  p.delta = a->pair_delta; p.d2 = a->pair_dist2; p.dist = a->pair_dist; p.dnorm = a->pair_dist_norm;
  p.bits = a->mask_bits; p.rc2 = a->cutoff * a->cutoff;
  p.B = a->batch; p.N = a->atoms; p.W = (a->atoms + 31) / 32; p.chunks = (a->atoms + 63) / 64;
  const long long units = (long long)p.B * p.N * p.chunks;
  const int grid = int(std::min<long long>((units + kWavesPerBlock - 1) / kWavesPerBlock, (long long)dev.num_cus * 32));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->scale_mode == MF_SCALE_RMS) {
    hipLaunchKernelGGL(rms_kernel, dim3(a->batch), dim3(kThreads), 0, s, a->coords, a->pad_mask, a->scale,
                       a->atoms);
    MF_HIP_CHECK(hipGetLastError());
  }
  if (a->gram == nullptr) hipLaunchKernelGGL(features_kernel<0>, dim3(grid), dim3(kThreads), 0, s, p);
  else if (a->pbc_radius == 1) hipLaunchKernelGGL(features_kernel<1>, dim3(grid), dim3(kThreads), 0, s, p);
  else hipLaunchKernelGGL(features_kernel<2>, dim3(grid), dim3(kThreads), 0, s, p);
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

/*
 * Radius (cutoff) neighbour mask with minimum image -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the pair distance of the reference's geometry adapters
 * (src/matterformer/geometry/adapters.py):
 *   periodic (gram != NULL)  :176-190  delta = f_i - f_j over the integer image
 *       offsets {-r..r}^3 (itertools.product order, :141-149); squared length
 *       under the lattice metric G = cell cell^T (lattice.py:94-100),
 *       d2 = delta^T G delta; the minimum over the images.
 *   non-periodic (gram == NULL) :98-99  d2 = (dx*dx + dy*dy) + dz*dz.
 * The fp32 evaluation order is fixed here (built with -ffp-contract=off):
 *   e   = delta + offset                      (per component)
 *   t_c = (G[c][0]*e0 + G[c][1]*e1) + G[c][2]*e2
 *   d2  = (e0*t_0 + e1*t_1) + e2*t_2
 * The reference evaluates the same quadratic form with einsum (its own order);
 * tests compare the two within float tolerance and this oracle with the HIP
 * kernel bit for bit.
 *
 * mask[i,j] = (d2_min(i,j) <= cutoff*cutoff), i == j included (d2 = 0), and 0
 * when i or j is padding.  Output: bits[b][i][w] bit t <-> j = 32 w + t, and
 * block_mask[b][bi][bj] = any bit set in the (block x block) tile.
 *
 * Pinned by: tests/test_oracle_radius.py (reference golden min-image
 * distances, the min-image KAT of tests/test_geometry.py:30-39, brute force
 * over a 5x5x5 image shell, symmetry).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_pair_d2(const float* xi, const float* xj, const float* G, int32_t pbc_radius) {
  const float d0 = xi[0] - xj[0];
  const float d1 = xi[1] - xj[1];
  const float d2v = xi[2] - xj[2];
  if (!G) {
    const float a = d0 * d0;
    const float b = d1 * d1;
    const float c = d2v * d2v;
    const float s = a + b;
    return s + c;
  }
  float best = INFINITY;
  for (int32_t o0 = -pbc_radius; o0 <= pbc_radius; ++o0)
    for (int32_t o1 = -pbc_radius; o1 <= pbc_radius; ++o1)
      for (int32_t o2 = -pbc_radius; o2 <= pbc_radius; ++o2) {
        const float e0 = d0 + (float)o0;
        const float e1 = d1 + (float)o1;
        const float e2 = d2v + (float)o2;
        float t[3];
        for (int c = 0; c < 3; ++c) {
          const float p0 = G[c * 3 + 0] * e0;
          const float p1 = G[c * 3 + 1] * e1;
          const float p2 = G[c * 3 + 2] * e2;
          const float s = p0 + p1;
          t[c] = s + p2;
        }
        const float q0 = e0 * t[0];
        const float q1 = e1 * t[1];
        const float q2 = e2 * t[2];
        const float s = q0 + q1;
        const float d2 = s + q2;
        if (d2 < best) best = d2;
      }
  return best;
}

void oracle_radius_mask(const float* coords, const float* gram, const uint8_t* pad_mask, int32_t B, int32_t N,
                        float cutoff, int32_t pbc_radius, int32_t block, uint32_t* bits, uint8_t* block_mask) {
  const int32_t W = (N + 31) / 32;
  const int32_t NB = (N + block - 1) / block;
  const float rc2 = cutoff * cutoff;
  memset(bits, 0, sizeof(uint32_t) * (size_t)B * N * W);
  if (block_mask) memset(block_mask, 0, (size_t)B * NB * NB);
  for (int32_t b = 0; b < B; ++b) {
    const float* x = coords + (int64_t)b * N * 3;
    const float* G = gram ? gram + (int64_t)b * 9 : 0;
    const uint8_t* pad = pad_mask ? pad_mask + (int64_t)b * N : 0;
    for (int32_t i = 0; i < N; ++i) {
      if (pad && pad[i]) continue;
      for (int32_t j = 0; j < N; ++j) {
        if (pad && pad[j]) continue;
        const float d2 = oracle_pair_d2(x + i * 3, x + j * 3, G, pbc_radius);
        if (d2 <= rc2) {
          bits[((int64_t)b * N + i) * W + j / 32] |= 1u << (j % 32);
          if (block_mask) block_mask[((int64_t)b * NB + i / block) * NB + j / block] = 1;
        }
      }
    }
  }
}

void oracle_pair_d2_matrix(const float* coords, const float* gram, int32_t B, int32_t N, int32_t pbc_radius,
                           float* d2) {
  for (int32_t b = 0; b < B; ++b) {
    const float* x = coords + (int64_t)b * N * 3;
    const float* G = gram ? gram + (int64_t)b * 9 : 0;
    for (int32_t i = 0; i < N; ++i)
      for (int32_t j = 0; j < N; ++j)
        d2[((int64_t)b * N + i) * N + j] = oracle_pair_d2(x + i * 3, x + j * 3, G, pbc_radius);
  }
}

/*
 * kNN brute force -- TEST INFRASTRUCTURE ONLY (CPU oracle, see oracle/__init__.py).
 *
 * The reference has no kNN in its active package; its only ancestor is the
 * legacy torch_cluster wrapper legacy/rapidash_v5/models/rapidash_utils.py:139-193
 * (knn / knn_graph, cdist + topk fallback, unspecified tie order).  This
 * restates the textbook algorithm with the reference's distance convention:
 *   delta = x_i - x_j                      (geometry/adapters.py:98)
 *   d2    = (dx*dx + dy*dy) + dz*dz        (adapters.py:99, square().sum(-1),
 *                                           fp32, each operation rounded; built
 *                                           with -ffp-contract=off)
 * For every valid atom i: the k valid atoms j != i (self included when
 * exclude_self == 0) with the smallest (d2, j), i.e. ties go to the lower
 * index.  dist = sqrtf(d2) (correctly rounded).  Slots beyond the number of
 * candidates get idx -1 and dist +inf; rows of padded atoms are all -1 / +inf.
 * pad_mask uses the reference's convention: nonzero = padding.
 *
 * Pinned by: tests/test_oracle_knn.py (bitwise agreement of d2 with the
 * reference adapter's pair_dist2 golden vectors, a numpy lexsort restatement,
 * hand-built ties and a uniform lattice).
 */
#include <math.h>
#include <stdint.h>

void oracle_knn(const float* coords, const uint8_t* pad_mask, int32_t B, int32_t N, int32_t K,
                int32_t exclude_self, int32_t* idx, float* dist, float* d2_scratch) {
  for (int32_t b = 0; b < B; ++b) {
    const float* x = coords + (int64_t)b * N * 3;
    const uint8_t* pad = pad_mask ? pad_mask + (int64_t)b * N : 0;
    for (int32_t i = 0; i < N; ++i) {
      int32_t* oi = idx + ((int64_t)b * N + i) * K;
      float* od = dist + ((int64_t)b * N + i) * K;
      for (int32_t s = 0; s < K; ++s) {
        oi[s] = -1;
        od[s] = INFINITY;
      }
      if (pad && pad[i]) continue;
      /* candidate distances; -1 marks excluded candidates */
      for (int32_t j = 0; j < N; ++j) {
        const int excluded = (pad && pad[j]) || (exclude_self && j == i);
        if (excluded) {
          d2_scratch[j] = -1.0f;
          continue;
        }
        const float dx = x[i * 3 + 0] - x[j * 3 + 0];
        const float dy = x[i * 3 + 1] - x[j * 3 + 1];
        const float dz = x[i * 3 + 2] - x[j * 3 + 2];
        const float xx = dx * dx;
        const float yy = dy * dy;
        const float zz = dz * dz;
        const float s = xx + yy;
        d2_scratch[j] = s + zz;
      }
      /* k rounds of selection of the smallest (d2, j) */
      for (int32_t s = 0; s < K; ++s) {
        int32_t best = -1;
        float bd = 0.0f;
        for (int32_t j = 0; j < N; ++j) {
          const float v = d2_scratch[j];
          if (v < 0.0f) continue;
          if (best < 0 || v < bd) { /* strict: equal keeps the lower j */
            best = j;
            bd = v;
          }
        }
        if (best < 0) break;
        oi[s] = best;
        od[s] = sqrtf(bd);
        d2_scratch[best] = -1.0f;
      }
    }
  }
}

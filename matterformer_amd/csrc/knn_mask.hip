// kNN neighbour lists -> the bit mask and 64-atom block mask of local
// attention (mf_knn_mask) on gfx950.
//
// The reference has no kNN attention; its trunk can only express one as an
// MHA block with a 0 / -inf attn_head_bias (src/matterformer/models/
// transformer.py:256-268).  This entry point turns the lists mf_knn returns
// into the mask layout mf_radius_attn reads, so kNN-local attention is that
// kernel over these bits:
//   mask[b, i, j] = valid_i && (j in idx[b, i, :] || (include_self && j == i))
// Integer work only; two small launches:
//   words   one thread per (b, i, 32-column word): scans the k indices of row i
//   blocks  one wave per (b, 64-row block, 64-column block): OR of its words
#include <algorithm>

#include "mf_common.h"

namespace mf {
namespace knnmask {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) words_kernel(const int32_t* __restrict__ idx,
                                                         const uint8_t* __restrict__ pad, uint32_t* __restrict__ bits,
                                                         int B, int N, int K, int W, int include_self) {
  const long long total = (long long)B * N * W;
  for (long long t = (long long)blockIdx.x * kThreads + threadIdx.x; t < total;
       t += (long long)gridDim.x * kThreads) {
    const long long row = t / W;  // b * N + i
    const int w = int(t - row * W);
    const int i = int(row % N);
    uint32_t word = 0;
    if (pad == nullptr || pad[row] == 0) {
      const int32_t* r = idx + row * K;
      for (int s = 0; s < K; ++s) {
        const int j = r[s];
        if (j >= 0 && j < N && (j >> 5) == w) word |= 1u << (j & 31);
      }
      if (include_self && (i >> 5) == w) word |= 1u << (i & 31);
    }
    bits[t] = word;
  }
}

// One wave per (b, 64-row block, 64-column block): lane r ORs the (at most
// two) words of row 64*bi + r that cover the column block, then one ballot.
__global__ void __launch_bounds__(kThreads) blocks_kernel(const uint32_t* __restrict__ bits,
                                                          uint8_t* __restrict__ block_mask, int B, int N, int W,
                                                          int NB) {
  const long long total = (long long)B * NB * NB;
  const int lane = threadIdx.x & 63;
  for (long long t = (long long)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); t < total;
       t += (long long)gridDim.x * (kThreads / 64)) {
    const int bj = int(t % NB);
    const int bi = int((t / NB) % NB);
    const long long b = t / ((long long)NB * NB);
    const int r = 64 * bi + lane;
    uint32_t any = 0;
    if (r < N) {
      const uint32_t* row = bits + ((long long)b * N + r) * W;
      any = row[2 * bj];
      if (2 * bj + 1 < W) any |= row[2 * bj + 1];
    }
    const unsigned long long hit = __ballot(any != 0);
    if (lane == 0) block_mask[t] = hit != 0 ? 1 : 0;
  }
}

}  // namespace knnmask
}  // namespace mf

extern "C" int mf_knn_mask(const mf_knn_mask_args* a, void* stream) {
  using namespace mf;
  using namespace mf::knnmask;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn_mask: args is NULL");
  if (!a->idx || !a->mask_bits) return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn_mask: idx and mask_bits must be non-NULL");
  if (a->batch < 0 || a->atoms < 0 || a->k < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_knn_mask: batch, atoms and k must be non-negative");
  if (a->batch == 0 || a->atoms == 0) return MF_OK;
  DeviceInfo dev;
  int st = device_info(&dev);
  if (st != MF_OK) return st;
  const int B = a->batch, N = a->atoms, W = (N + 31) / 32, NB = (N + 63) / 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long long words = (long long)B * N * W;
  const int grid1 = int(std::min<long long>((words + kThreads - 1) / kThreads, (long long)dev.num_cus * 16));
  hipLaunchKernelGGL(words_kernel, dim3(grid1), dim3(kThreads), 0, s, a->idx, a->pad_mask, a->mask_bits, B, N,
                     a->k, W, a->include_self != 0 ? 1 : 0);
  MF_HIP_CHECK(hipGetLastError());
  if (a->block_mask) {
    const long long tiles = (long long)B * NB * NB;
    const int grid2 = int(std::min<long long>((tiles + 3) / 4, (long long)dev.num_cus * 16));
    hipLaunchKernelGGL(blocks_kernel, dim3(grid2), dim3(kThreads), 0, s, a->mask_bits, a->block_mask, B, N, W, NB);
    MF_HIP_CHECK(hipGetLastError());
  }
  return MF_OK;
}

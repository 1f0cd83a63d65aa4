// Shared device/host helpers for the gfx950 kernels of libmf_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/mf_capi.h"

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local last error, see mf_last_error()).
// ---------------------------------------------------------------------------
namespace mf {

void set_last_error(const std::string& msg);
int fail(int status, const std::string& msg);

// Per-device properties cached on first use.
struct DeviceInfo {
  int device = -1;
  int num_cus = 0;
  int max_lds_per_block = 0;
};
int device_info(DeviceInfo* out);

// hipFuncSetAttribute(kernel, MaxDynamicSharedMemorySize, bytes) once per
// (kernel, current device, bytes), under a lock: safe from several host threads
// and on every device the library runs on.
int ensure_dynamic_lds(const void* kernel, int bytes);

// Register-resident simplicial kernels for 16-bit operands (simplicial_fast.hip).
int simplicial_fast_capacity(int head_dim);
size_t simplicial_fast_workspace_bytes(int batch, int heads, int tokens);
int simplicial_fast_launch(const mf_simplicial_fwd_args* a, void* workspace, int num_cus, hipStream_t stream);
constexpr int kSimplicialFastMaxBatch = 1024;  // molecules per launch slice

// Pair-flash simplicial kernel for 16-bit operands (simplicial_pair.hip):
// one launch per slice of simplicial_pair_max_batch molecules; its claim
// region (simplicial_pair_workspace_bytes) holds the unit-claim counter,
// 0 before the first launch and left 0 by every launch.
bool simplicial_pair_serves(int tokens, int head_dim, int dtype);
int simplicial_pair_max_batch(int tokens);
size_t simplicial_pair_workspace_bytes(int batch, int tokens);
int simplicial_pair_launch(const mf_simplicial_fwd_args* a, void* claims, int num_cus, hipStream_t stream);

// Pair-formulation backward for bf16 operands (simplicial_pair_bwd.hip): it
// serves every molecule with at most simplicial_pair_bwd_max_tokens() valid
// queries and keys and leaves the others untouched.
// It needs simplicial_pair_bwd_workspace_bytes() of 256-byte aligned
// workspace (a plan of units, served flags, atom lists and partial
// sums); after a launch simplicial_pair_bwd_served() points at one int per
// molecule, nonzero when the pair kernel computed its gradients.
bool simplicial_pair_bwd_serves(const mf_simplicial_bwd_args* a);
int simplicial_pair_bwd_max_tokens();
size_t simplicial_pair_bwd_workspace_bytes(int batch, int heads);
const int* simplicial_pair_bwd_served(const mf_simplicial_bwd_args* a);
const int* simplicial_pair_bwd_unserved_count(const mf_simplicial_bwd_args* a);  // molecules left over
int simplicial_pair_bwd_launch(const mf_simplicial_bwd_args* a, hipStream_t stream);

#define MF_HIP_CHECK(expr)                                                     \
  do {                                                                         \
    hipError_t mf_err_ = (expr);                                               \
    if (mf_err_ != hipSuccess)                                                 \
      return ::mf::fail(MF_ERR_HIP, std::string(#expr) + ": " +                \
                                        hipGetErrorString(mf_err_));           \
  } while (0)

}  // namespace mf

// ---------------------------------------------------------------------------
// Device-side vector types and MFMA wrappers (CDNA4 / gfx950, wave64).
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 mf_bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 mf_f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float mf_f32x4;

namespace mf {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// Sum over the 16 lanes that share lane>>4 (an MFMA "row group").
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ds_read_b64_tr_b16 (gfx950): four 16-bit elements, transposed within each
// group of 16 lanes: lane 4a + c receives element c of the 8-byte pieces
// addressed by lanes 4e + a of its group, e = 0..3 in order.  p must be
// 8-byte aligned LDS.
template <typename T>
__device__ __forceinline__ auto read_tr16(const T* p) {
  typedef __attribute__((__vector_size__(4 * sizeof(T)))) T Op4;
  typedef short s4 __attribute__((ext_vector_type(4)));
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4*)(reinterpret_cast<uintptr_t>(p)));
  return __builtin_bit_cast(Op4, v);
}

// Element traits: 16-bit types use the K=32 MFMA (8 K-elements per lane),
// fp32 uses the K=4 MFMA (1 K-element per lane).  Both produce the same
// 16x16 fp32 accumulator layout: lane l holds C[4*(l>>4)+r][l&15], r=0..3.
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  static constexpr int kSize = 2;
  static constexpr int kKPerMfma = 32;
  static constexpr int kKPerLane = 8;
  using Operand = mf_bf16x8;
  __device__ static __forceinline__ float to_f32(__bf16 x) { return static_cast<float>(x); }
  __device__ static __forceinline__ __bf16 from_f32(float x) { return static_cast<__bf16>(x); }
  __device__ static __forceinline__ mf_f32x4 mma(Operand a, Operand b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<_Float16> {
  static constexpr int kSize = 2;
  static constexpr int kKPerMfma = 32;
  static constexpr int kKPerLane = 8;
  using Operand = mf_f16x8;
  __device__ static __forceinline__ float to_f32(_Float16 x) { return static_cast<float>(x); }
  __device__ static __forceinline__ _Float16 from_f32(float x) { return static_cast<_Float16>(x); }
  __device__ static __forceinline__ mf_f32x4 mma(Operand a, Operand b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<float> {
  static constexpr int kSize = 4;
  static constexpr int kKPerMfma = 4;
  static constexpr int kKPerLane = 1;
  using Operand = float;
  __device__ static __forceinline__ float to_f32(float x) { return x; }
  __device__ static __forceinline__ float from_f32(float x) { return x; }
  __device__ static __forceinline__ mf_f32x4 mma(Operand a, Operand b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

}  // namespace mf

// Per-token glue of the packed AdaLN trunk on gfx950: the valid atoms of a
// padded batch are the rows of one [T, C] matrix, and these kernels do the
// work the reference's AdaLNBlock does elementwise around its attention and
// MLP (src/matterformer/models/transformer.py:296-316), plus the reshapes
// between the packed rows and the [B, H, W, D] head layout the attention
// kernels read (SimplicialAttention._split_heads / _merge_heads,
// simplicial_attention.py).
//
//   mf_adaln_rows        x' = x + gate[mol] * y                   (residual)
//                        h  = LN(x') * (1 + scale[mol]) + shift[mol]
//                        either half optional; one wave per row.
//   mf_rows_to_heads     [T, P*H*D] -> [P, B, H, W, D] through a slot map
//                        (source row of (b, w), -1 = zero), part 0 scaled.
//   mf_heads_to_rows     [B, H, W, D] -> [T, H*D] through a row index.
//
// Rounding follows the torch expressions the reference evaluates in the
// activation dtype T: every product and sum is rounded to T
// (x + round(gate * y); round(round(LN) * round(1 + scale)) + shift, rounded),
// LayerNorm (no affine, nn.LayerNorm with elementwise_affine=False) in fp32
// with its output rounded to T.  This file is built without FMA contraction.
#include <algorithm>
#include <cmath>

#include "mf_common.h"

namespace mf {
namespace rows {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 4;  // C <= 64 lanes * 8 * 4 = 2048

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  return Elem<T>::to_f32(Elem<T>::from_f32(v));
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elem<T>::to_f32(e[i]);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    uint4 u;
    T* e = reinterpret_cast<T*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = Elem<T>::from_f32(v[i]);
    *reinterpret_cast<uint4*>(p) = u;
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

template <typename T>
__device__ __forceinline__ void zero_store8(T* p) {
  float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  store8(p, z);
}

struct AdaParams {
  const void* x;
  const void* y;
  const void* gate;
  const void* shift;
  const void* scale;
  const int32_t* mol;
  void* x_out;
  void* h_out;
  float eps;
  int T, C, stride;
};

// One wave per row; lane l holds the 8-element groups l, l + 64, ... of it
// (CH = ceil(C / 512) groups per lane).
template <typename T, int CH>
__global__ void __launch_bounds__(kThreads) adaln_rows_kernel(AdaParams p) {
  const int lane = threadIdx.x & 63;
  const long long t = (long long)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (t >= p.T) return;
  const int groups = p.C / 8;
  const long long m = p.mol[t];
  float v[CH][8];
  const T* x = static_cast<const T*>(p.x) + t * p.C;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int g = lane + 64 * c;
    if (g < groups) load8(x + 8 * g, v[c]);
  }
  // every global load of the row is issued before the first use: one memory round trip per wave
  float sh[CH][8], sc[CH][8];
  if (p.shift) {
    const T* shift = static_cast<const T*>(p.shift) + m * p.stride;
    const T* scale = static_cast<const T*>(p.scale) + m * p.stride;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int g = lane + 64 * c;
      if (g < groups) {
        load8(shift + 8 * g, sh[c]);
        load8(scale + 8 * g, sc[c]);
      }
    }
  }
  if (p.y) {
    const T* y = static_cast<const T*>(p.y) + t * p.C;
    const T* gate = static_cast<const T*>(p.gate) + m * p.stride;
    float yv[CH][8], gv[CH][8];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int g = lane + 64 * c;
      if (g < groups) {
        load8(y + 8 * g, yv[c]);
        load8(gate + 8 * g, gv[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int g = lane + 64 * c;
      if (g >= groups) continue;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float prod = rnd<T>(gv[c][i] * yv[c][i]);
        v[c][i] = rnd<T>(v[c][i] + prod);
      }
      store8(static_cast<T*>(p.x_out) + t * p.C + 8 * g, v[c]);
    }
  }
  if (!p.shift) return;
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
    if (lane + 64 * c < groups)
#pragma unroll
      for (int i = 0; i < 8; ++i) s += v[c][i];
  const float mean = wave_sum(s) / float(p.C);
  float q = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
    if (lane + 64 * c < groups)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[c][i] - mean;
        q += d * d;
      }
  const float var = wave_sum(q) / float(p.C);
  const float rstd = 1.0f / sqrtf(var + p.eps);
  T* h = static_cast<T*>(p.h_out) + t * p.C;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int g = lane + 64 * c;
    if (g >= groups) continue;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float n = rnd<T>((v[c][i] - mean) * rstd);
      const float one_plus = rnd<T>(1.0f + sc[c][i]);
      const float prod = rnd<T>(n * one_plus);
      o[i] = prod + sh[c][i];
    }
    store8(h + 8 * g, o);
  }
}

struct HeadsParams {
  const void* src;
  const int32_t* index;  // slot map (rows -> heads) or row index (heads -> rows)
  void* dst;
  float scale0;
  int T, P, B, H, W, D;
};

// Thread per 8 consecutive elements of the destination [P, B, H, W, D].
// Index arithmetic in 32 bits: the host checks every element count < 2^31.
template <typename TS, typename TD>
__global__ void __launch_bounds__(kThreads) rows_to_heads_kernel(HeadsParams p) {
  const unsigned d8 = unsigned(p.D) / 8u;
  const unsigned total = unsigned(p.P) * p.B * p.H * p.W * d8;
  const unsigned i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  unsigned r = i / d8;
  const int d = int(i - r * d8) * 8;
  const unsigned r2 = r / unsigned(p.W);
  const int w = int(r - r2 * unsigned(p.W));
  const unsigned r3 = r2 / unsigned(p.H);
  const int h = int(r2 - r3 * unsigned(p.H));
  const unsigned part = r3 / unsigned(p.B);
  const int b = int(r3 - part * unsigned(p.B));
  TD* out = static_cast<TD*>(p.dst) + size_t(i) * 8;
  const int t = p.index[b * p.W + w];
  if (t < 0) {
    zero_store8(out);
    return;
  }
  float v[8];
  load8(static_cast<const TS*>(p.src) + unsigned(t) * unsigned(p.P * p.H * p.D) + (part * p.H + h) * p.D + d, v);
  if (part == 0 && p.scale0 != 1.0f) {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = rnd<TS>(v[k] * p.scale0);
  }
  store8(out, v);
}

// Thread per 8 consecutive elements of the destination row [T, H*D].
template <typename TS, typename TD>
__global__ void __launch_bounds__(kThreads) heads_to_rows_kernel(HeadsParams p) {
  const unsigned row8 = unsigned(p.H * p.D) / 8u;
  const unsigned total = unsigned(p.T) * row8;
  const unsigned i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const unsigned t = i / row8;
  const int c = int(i - t * row8) * 8;
  const int h = c / p.D;
  const int d = c - h * p.D;
  const unsigned bw = unsigned(p.index[t]);
  const unsigned b = bw / unsigned(p.W);
  const unsigned w = bw - b * unsigned(p.W);
  float v[8];
  load8(static_cast<const TS*>(p.src) + ((b * p.H + h) * p.W + w) * p.D + d, v);
  store8(static_cast<TD*>(p.dst) + size_t(i) * 8, v);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

template <bool TO_HEADS, typename TS, typename TD>
void launch_kernel(dim3 grid, hipStream_t s, const HeadsParams& hp) {
  if constexpr (TO_HEADS) hipLaunchKernelGGL((rows_to_heads_kernel<TS, TD>), grid, dim3(kThreads), 0, s, hp);
  else hipLaunchKernelGGL((heads_to_rows_kernel<TS, TD>), grid, dim3(kThreads), 0, s, hp);
}

template <bool TO_HEADS, typename TS>
int launch_heads(int dst_dtype, const HeadsParams& hp, long long total, hipStream_t s) {
  const dim3 grid(unsigned((total + kThreads - 1) / kThreads));
  switch (dst_dtype) {
    case MF_DTYPE_BF16: launch_kernel<TO_HEADS, TS, __bf16>(grid, s, hp); break;
    case MF_DTYPE_F16: launch_kernel<TO_HEADS, TS, _Float16>(grid, s, hp); break;
    default: launch_kernel<TO_HEADS, TS, float>(grid, s, hp); break;
  }
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

template <bool TO_HEADS>
int dispatch_heads(int src_dtype, int dst_dtype, const HeadsParams& hp, long long total, hipStream_t s) {
  switch (src_dtype) {
    case MF_DTYPE_BF16: return launch_heads<TO_HEADS, __bf16>(dst_dtype, hp, total, s);
    case MF_DTYPE_F16: return launch_heads<TO_HEADS, _Float16>(dst_dtype, hp, total, s);
    default: return launch_heads<TO_HEADS, float>(dst_dtype, hp, total, s);
  }
}

template <typename T>
void launch_adaln(int chunks, dim3 grid, hipStream_t s, const AdaParams& p) {
  switch (chunks) {
    case 1: hipLaunchKernelGGL((adaln_rows_kernel<T, 1>), grid, dim3(kThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((adaln_rows_kernel<T, 2>), grid, dim3(kThreads), 0, s, p); break;
    case 3: hipLaunchKernelGGL((adaln_rows_kernel<T, 3>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((adaln_rows_kernel<T, 4>), grid, dim3(kThreads), 0, s, p); break;
  }
}

bool valid_dtype(int d) { return d == MF_DTYPE_F32 || d == MF_DTYPE_F16 || d == MF_DTYPE_BF16; }

}  // namespace rows
}  // namespace mf

extern "C" int mf_adaln_rows(const mf_adaln_rows_args* a, void* stream) {
  using namespace mf;
  using namespace mf::rows;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: args is NULL");
  if (a->tokens < 0 || a->channels <= 0 || a->batch < 0 || a->mod_stride < 0)
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: sizes must be non-negative (channels positive)");
  if (!valid_dtype(a->dtype)) return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: bad dtype");
  if (!a->x || !a->mol) return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: x and mol must be non-NULL");
  if (a->y && (!a->gate || !a->x_out))
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: a residual (y) needs gate and x_out");
  if (a->shift && (!a->scale || !a->h_out))
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: a modulated output (shift) needs scale and h_out");
  if (!a->y && !a->shift) return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: nothing to compute");
  if (!(a->eps >= 0.0f)) return fail(MF_ERR_INVALID_ARGUMENT, "mf_adaln_rows: eps must be non-negative");
  if (a->channels % 8 != 0 || a->channels > 64 * 8 * kMaxChunks || a->mod_stride % 8 != 0)
    return fail(MF_ERR_UNSUPPORTED, "mf_adaln_rows: channels (and mod_stride) must be multiples of 8, channels <= 2048");
  for (const void* ptr : {a->x, a->y, a->gate, a->shift, a->scale, static_cast<const void*>(a->x_out),
                          static_cast<const void*>(a->h_out)})
    if (ptr && !aligned16(ptr)) return fail(MF_ERR_UNSUPPORTED, "mf_adaln_rows: operands must be 16-byte aligned");
  if (a->tokens == 0) return MF_OK;
  AdaParams p{a->x, a->y, a->gate, a->shift, a->scale, a->mol, a->x_out, a->h_out, a->eps,
              a->tokens, a->channels, a->mod_stride};
  const dim3 grid(unsigned((a->tokens + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = (a->channels + 511) / 512;
  switch (a->dtype) {
    case MF_DTYPE_BF16: launch_adaln<__bf16>(chunks, grid, s, p); break;
    case MF_DTYPE_F16: launch_adaln<_Float16>(chunks, grid, s, p); break;
    default: launch_adaln<float>(chunks, grid, s, p); break;
  }
  MF_HIP_CHECK(hipGetLastError());
  return MF_OK;
}

static int check_heads(const char* name, const void* src, const int32_t* index, const void* dst, int T, int P, int B,
                       int H, int W, int D, int sd, int dd) {
  using namespace mf;
  using namespace mf::rows;
  const std::string n(name);
  if (!src || !index || !dst) return fail(MF_ERR_INVALID_ARGUMENT, n + ": pointers must be non-NULL");
  if (T < 0 || P <= 0 || B < 0 || H <= 0 || W < 0 || D <= 0)
    return fail(MF_ERR_INVALID_ARGUMENT, n + ": bad sizes");
  if (!valid_dtype(sd) || !valid_dtype(dd)) return fail(MF_ERR_INVALID_ARGUMENT, n + ": bad dtype");
  if (D % 8 != 0) return fail(MF_ERR_UNSUPPORTED, n + ": head_dim must be a multiple of 8");
  if (!aligned16(src) || !aligned16(dst)) return fail(MF_ERR_UNSUPPORTED, n + ": operands must be 16-byte aligned");
  const long long heads_elems = (long long)P * B * H * W * D, rows_elems = (long long)T * P * H * D;
  if (heads_elems >= (1ll << 31) || rows_elems >= (1ll << 31))
    return fail(MF_ERR_UNSUPPORTED, n + ": more than 2^31 - 1 elements");
  return MF_OK;
}

extern "C" int mf_rows_to_heads(const mf_rows_to_heads_args* a, void* stream) {
  using namespace mf;
  using namespace mf::rows;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_rows_to_heads: args is NULL");
  int st = check_heads("mf_rows_to_heads", a->rows, a->slot, a->heads, a->tokens, a->parts, a->batch, a->heads_count,
                       a->width, a->head_dim, a->src_dtype, a->dst_dtype);
  if (st != MF_OK) return st;
  if (!std::isfinite(a->first_part_scale))
    return fail(MF_ERR_INVALID_ARGUMENT, "mf_rows_to_heads: first_part_scale must be finite");
  const long long total = (long long)a->parts * a->batch * a->heads_count * a->width * (a->head_dim / 8);
  if (total == 0) return MF_OK;
  HeadsParams p{a->rows, a->slot, a->heads, a->first_part_scale, a->tokens, a->parts, a->batch, a->heads_count,
                a->width, a->head_dim};
  return dispatch_heads<true>(a->src_dtype, a->dst_dtype, p, total, static_cast<hipStream_t>(stream));
}

extern "C" int mf_heads_to_rows(const mf_heads_to_rows_args* a, void* stream) {
  using namespace mf;
  using namespace mf::rows;
  if (a == nullptr) return fail(MF_ERR_INVALID_ARGUMENT, "mf_heads_to_rows: args is NULL");
  int st = check_heads("mf_heads_to_rows", a->heads, a->row_index, a->rows, a->tokens, 1, a->batch, a->heads_count,
                       a->width, a->head_dim, a->src_dtype, a->dst_dtype);
  if (st != MF_OK) return st;
  const long long total = (long long)a->tokens * a->heads_count * a->head_dim / 8;
  if (total == 0) return MF_OK;
  HeadsParams p{a->heads, a->row_index, a->rows, 1.0f, a->tokens, 1, a->batch, a->heads_count, a->width, a->head_dim};
  return dispatch_heads<false>(a->src_dtype, a->dst_dtype, p, total, static_cast<hipStream_t>(stream));
}

// Measurement program (not part of libmf_hip.so): what bounds the pair loop of
// simplicial_pair.hip on gfx950.
//
// 1. The kernel's own pair_loop<DP = 64, QT, kFast> on synthetic fp16 operands
//    staged in LDS (nk = 44 keys, 48 query rows), repeated 200 times per wave,
//    at one and two workgroups (4 waves each) per CU: nanoseconds per
//    iteration per SIMD and per MFMA.
// 2. Instruction throughput on one SIMD: v_mfma_f32_16x16x32_f16 alone, with
//    K independent v_pk_mul_f16 after each, and v_exp_f32 / v_pk_mul_f16
//    alone, eight distinct A/B operand sets loaded from memory (inline asm,
//    fixed order), at one and two waves per SIMD.
// Cycles are quoted at the 2.4 GHz peak engine clock (ns x 2.4).
//
// Build and run: make -C matterformer_amd/csrc/probes && matterformer_amd/csrc/probes/pair_loop_probe
#include "../simplicial_pair.hip"

#include <cstdio>

namespace mf {
void set_last_error(const std::string&) {}
int fail(int s, const std::string&) { return s; }
}  // namespace mf
using namespace mf;
using namespace mf::spair;

__device__ __forceinline__ uint16_t probe_half(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352dU; x ^= x >> 15; x *= 0x846ca68bU; x ^= x >> 16;
  return __builtin_bit_cast(uint16_t, _Float16((float(x & 0xffff) / 65536.0f - 0.5f)));
}

template <int QT, int OCC>
__global__ void __launch_bounds__(256, OCC) loop_kernel(float* out, int nk, int reps) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  using Ly = Lay<64>;
  uint16_t* s16 = reinterpret_cast<uint16_t*>(smem);
  const int tid = threadIdx.x;
  for (int i = tid; i < Ly::kPV / 2; i += 256) {
    const int row = (i * 2 % (kCap * Ly::RB)) / Ly::RB;
    s16[i] = row < nk ? probe_half(i * 7919u + blockIdx.x) : 0;
  }
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6, g = lane >> 4, r16 = lane & 15;
  uint4 qop[3][2];
  for (int qt = 0; qt < 3; ++qt)
    for (int c = 0; c < 2; ++c)
      qop[qt][c] = *reinterpret_cast<const uint4*>(smem + Ly::kQ + (16 * qt + r16) * Ly::RB + c * 64 + g * 16);
  mf_f32x4 O[4][3], L[3];
  float mloc[3], negm[3];
  for (int qt = 0; qt < 3; ++qt) {
    L[qt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
    mloc[qt] = negm[qt] = 0.f;
    for (int dt = 0; dt < 4; ++dt) O[dt][qt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int r = 0; r < reps; ++r)
    pair_loop<64, QT, kFast, false, false>(smem, nk, nk, qop, negm, 1.0f, O, L, mloc, wave, g, r16);
  float acc = 0.f;
  for (int qt = 0; qt < 3; ++qt) {
    acc += L[qt][0];
    for (int dt = 0; dt < 4; ++dt) acc += O[dt][qt][0];
  }
  out[blockIdx.x * 256 + tid] = acc;
}

template <int QT, int OCC>
void run_loop(float* dout, int cus) {
  const int nk = 44, reps = 200;
  auto k = loop_kernel<QT, OCC>;
  const int lds = Lay<64>::kTotal;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  hipLaunchKernelGGL(k, dim3(cus * OCC), dim3(256), lds, 0, dout, nk, 2);
  (void)hipDeviceSynchronize();
  (void)hipEventRecord(a);
  hipLaunchKernelGGL(k, dim3(cus * OCC), dim3(256), lds, 0, dout, nk, reps);
  (void)hipEventRecord(b);
  (void)hipEventSynchronize(b);
  float ms;
  (void)hipEventElapsedTime(&ms, a, b);
  const int nkt = (nk + 15) / 16, njp = (nk + 1) / 2;
  const double iters = double(nkt * njp) / 4.0 * reps * OCC;  // iterations per SIMD
  const double ns = ms * 1e6 / iters;
  const int mfma = QT * 9;  // GEMM1 4 QT, GEMM2 4 QT, row sums QT
  printf("pair_loop QT=%d, %d workgroup(s)/CU (%d wave(s)/SIMD): %.1f ns/iteration/SIMD = %.0f cycles, %.1f per MFMA\n",
         QT, OCC, OCC, ns, ns * 2.4, ns * 2.4 / mfma);
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
#define PROBE_MF(c, a, b) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b))
#define PROBE_PK(x) asm volatile("v_pk_mul_f16 %0, %0, %1" : "+v"(x) : "v"(m))
#define PROBE_EX(x) asm volatile("v_exp_f32 %0, %0" : "+v"(x))

// MODE 0: 8 MFMA with K pk_mul after each; 1: 16 pk_mul; 2: 16 exp
template <int MODE, int K>
__global__ void __launch_bounds__(256) isa_kernel(const h8* __restrict__ src, float* out, int iters) {
  const int t = threadIdx.x;
  h8 a0 = src[t], a1 = src[t + 256], a2 = src[t + 512], a3 = src[t + 768];
  h8 a4 = src[t + 1024], a5 = src[t + 1280], a6 = src[t + 1536], a7 = src[t + 1792];
  h8 b0 = src[t + 2048], b1 = src[t + 2304], b2 = src[t + 2560], b3 = src[t + 2816];
  h8 b4 = src[t + 3072], b5 = src[t + 3328], b6 = src[t + 3584], b7 = src[t + 3840];
  f4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
  uint32_t m = 0x3c003c00u;
  uint32_t y0 = t, y1 = t + 1, y2 = t + 2, y3 = t + 3, y4 = t + 4, y5 = t + 5, y6 = t + 6, y7 = t + 7;
  uint32_t y8 = t + 8, y9 = t + 9, y10 = t + 10, y11 = t + 11, y12 = t + 12, y13 = t + 13, y14 = t + 14, y15 = t + 15;
  float x0 = 0.001f * t, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5, x6 = x0 + 6, x7 = x0 + 7;
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE == 0) {
      PROBE_MF(c0, a0, b0); if (K > 0) PROBE_PK(y0); if (K > 1) PROBE_PK(y1); if (K > 2) PROBE_PK(y2);
      PROBE_MF(c1, a1, b1); if (K > 0) PROBE_PK(y3); if (K > 1) PROBE_PK(y4); if (K > 2) PROBE_PK(y5);
      PROBE_MF(c2, a2, b2); if (K > 0) PROBE_PK(y6); if (K > 1) PROBE_PK(y7); if (K > 2) PROBE_PK(y8);
      PROBE_MF(c3, a3, b3); if (K > 0) PROBE_PK(y9); if (K > 1) PROBE_PK(y10); if (K > 2) PROBE_PK(y11);
      PROBE_MF(c4, a4, b4); if (K > 0) PROBE_PK(y12); if (K > 1) PROBE_PK(y13); if (K > 2) PROBE_PK(y14);
      PROBE_MF(c5, a5, b5); if (K > 0) PROBE_PK(y15); if (K > 1) PROBE_PK(y0); if (K > 2) PROBE_PK(y1);
      PROBE_MF(c6, a6, b6); if (K > 0) PROBE_PK(y2); if (K > 1) PROBE_PK(y3); if (K > 2) PROBE_PK(y4);
      PROBE_MF(c7, a7, b7); if (K > 0) PROBE_PK(y5); if (K > 1) PROBE_PK(y6); if (K > 2) PROBE_PK(y7);
    } else if constexpr (MODE == 1) {
      PROBE_PK(y0); PROBE_PK(y1); PROBE_PK(y2); PROBE_PK(y3); PROBE_PK(y4); PROBE_PK(y5); PROBE_PK(y6); PROBE_PK(y7);
      PROBE_PK(y8); PROBE_PK(y9); PROBE_PK(y10); PROBE_PK(y11); PROBE_PK(y12); PROBE_PK(y13); PROBE_PK(y14);
      PROBE_PK(y15);
    } else {
      PROBE_EX(x0); PROBE_EX(x1); PROBE_EX(x2); PROBE_EX(x3); PROBE_EX(x4); PROBE_EX(x5); PROBE_EX(x6); PROBE_EX(x7);
      PROBE_EX(x0); PROBE_EX(x1); PROBE_EX(x2); PROBE_EX(x3); PROBE_EX(x4); PROBE_EX(x5); PROBE_EX(x6); PROBE_EX(x7);
    }
  }
  float s = c0[0] + c1[1] + c2[2] + c3[3] + c4[0] + c5[1] + c6[2] + c7[3] + x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7;
  s += float(y0 ^ y1 ^ y2 ^ y3 ^ y4 ^ y5 ^ y6 ^ y7 ^ y8 ^ y9 ^ y10 ^ y11 ^ y12 ^ y13 ^ y14 ^ y15);
  out[blockIdx.x * 256 + t] = s;
}

template <int MODE, int K>
void run_isa(const char* name, const h8* src, float* d, int cus, int wps) {
  const int iters = 4000;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  hipLaunchKernelGGL((isa_kernel<MODE, K>), dim3(cus * wps), dim3(256), 0, 0, src, d, 10);
  (void)hipDeviceSynchronize();
  (void)hipEventRecord(e0);
  hipLaunchKernelGGL((isa_kernel<MODE, K>), dim3(cus * wps), dim3(256), 0, 0, src, d, iters);
  (void)hipEventRecord(e1);
  (void)hipEventSynchronize(e1);
  float ms;
  (void)hipEventElapsedTime(&ms, e0, e1);
  const double cyc = ms * 1e-3 * 2.4e9 / (double(iters) * wps);
  const int n = MODE == 0 ? 8 : 16;
  printf("%-34s %d wave(s)/SIMD: %.1f cycles per 16 instructions' group -> %.2f per %s\n", name, wps, cyc,
         cyc / n, MODE == 0 ? "MFMA" : "instruction");
}

int main() {
  hipDeviceProp_t prop;
  (void)hipGetDeviceProperties(&prop, 0);
  const int cus = prop.multiProcessorCount;
  printf("device %s, %d CUs\n", prop.gcnArchName, cus);
  float* d;
  (void)hipMalloc(&d, size_t(cus) * 4 * 256 * 4);
  run_loop<3, 1>(d, cus);
  run_loop<3, 2>(d, cus);
  run_loop<2, 1>(d, cus);
  run_loop<2, 2>(d, cus);
  h8* src;
  (void)hipMalloc(&src, 4096 * sizeof(h8));
  (void)hipMemset(src, 0, 4096 * sizeof(h8));
  for (int w : {1, 2}) {
    run_isa<0, 0>("8 MFMA (distinct A, B)", src, d, cus, w);
    run_isa<0, 1>("8 MFMA + 1 v_pk_mul_f16 each", src, d, cus, w);
    run_isa<0, 2>("8 MFMA + 2 v_pk_mul_f16 each", src, d, cus, w);
    run_isa<0, 3>("8 MFMA + 3 v_pk_mul_f16 each", src, d, cus, w);
    run_isa<1, 0>("16 v_pk_mul_f16", src, d, cus, w);
    run_isa<2, 0>("16 v_exp_f32", src, d, cus, w);
  }
  return 0;
}

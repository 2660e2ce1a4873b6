// Compute-only model of the wide projection kernel (k_linear_wide): per wave
// and group it runs the kernel's arithmetic on a 32 x 64 output tile (two
// 32x32 tiles, K = 64) with operands in registers -- no memory, no LDS, no
// barriers.  Its rate is the ceiling that the bit-exact group-64 rescale leaves
// the kernel: the i8 dots are 128 MFMA cycles per wave and group, the rest is
// the fp32 rescale (conversion, product, t, s) of 2048 outputs.
//
// Variants (the numbers in brackets are this file's template argument MODE):
//   [0] the kernel's form: two v_mfma_i32_32x32x32_i8 per tile, conversion
//       and product by v_mfma_f32_32x32x1_2b_f32, t and s on the VALU;
//   [3] conversion by v_cvt_f32_i32 instead of the K=1 MFMA;
//   [4] conversion and product by v_mfma_f32_4x4x1_16b_f32 (4-row slices);
//   [1] software-pipelined: group g-1's rescale between group g's MFMAs,
//       v_cvt conversion, 4x4x1 products;
//   [2] the same with 4x4x1 conversion.
// Output: SIMD cycles per wave and group, and the int8 rate that gives.
// Build and run: make -C decider-engine_amd/microbench && decider-engine_amd/microbench/wide_inner
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#pragma clang fp contract(off)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e = (x);                                                       \
    if (e != hipSuccess) {                                                    \
      printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__);   \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

constexpr int kMagicBits = 0x4B400000;
constexpr float kMagic = 12582912.0f;

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v32f mfma_k1(float a, float b, v32f c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_k1_4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v32f concat(v16i lo, v16i hi) {
  v16f a = __builtin_bit_cast(v16f, lo), b = __builtin_bit_cast(v16f, hi);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20,
                                 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
}

template <int MODE>
__global__ __launch_bounds__(256) void k_inner(int iters, long long* cyc, float* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v4i a0 = {lane, 3, 5, 7}, a1 = {lane * 3, 1, 2, 3};
  v4i b00 = {1, lane, 2, 3}, b01 = {4, 5, lane, 7}, b10 = {9, 8, 7, lane}, b11 = {lane, lane, 1, 1};
  float x = 0.001f * lane, w = 0.002f * lane;
  const float xu[4] = {x, x * 2, x * 3, x * 4};
  v16i cinit, zero16i;
  for (int i = 0; i < 16; ++i) {
    cinit[i] = kMagicBits;
    zero16i[i] = 0;
  }
  v32f zero32;
  for (int i = 0; i < 32; ++i) zero32[i] = 0.0f;
  const v4f zero4 = {0, 0, 0, 0};
  v32f s = zero32;
  v16i dacc[2] = {MODE == 2 ? cinit : zero16i, MODE == 2 ? cinit : zero16i};
  const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    asm volatile("" : "+v"(a0), "+v"(a1), "+v"(b00), "+v"(b01), "+v"(b10), "+v"(b11), "+v"(x), "+v"(w));
    if constexpr (MODE == 0 || MODE == 3 || MODE == 4) {
      const v16i c = MODE == 3 ? zero16i : cinit;
      v16i d0 = mfma_i8(a0, b00, c), d1 = mfma_i8(a0, b10, c);
      d0 = mfma_i8(a1, b01, d0);
      d1 = mfma_i8(a1, b11, d1);
      if constexpr (MODE == 0) {
        const v32f dv = mfma_k1(-kMagic, 1.0f, concat(d0, d1));
        const v32f pv = mfma_k1(x, w, zero32);
        s = s + dv * pv;
      } else if constexpr (MODE == 3) {
        const v32f pv = mfma_k1(x, w, zero32);
        v32f dv;
        for (int i = 0; i < 16; ++i) {
          dv[i] = (float)d0[i];
          dv[16 + i] = (float)d1[i];
        }
        s = s + dv * pv;
      } else {
        const v16i dd[2] = {d0, d1};
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            v4i bits;
            for (int i = 0; i < 4; ++i) bits[i] = dd[c2][4 * u + i];
            const v4f dv = mfma_k1_4(-kMagic, 1.0f, __builtin_bit_cast(v4f, bits));
            const v4f pv = mfma_k1_4(xu[u], w, zero4);
            for (int i = 0; i < 4; ++i) s[16 * c2 + 4 * u + i] = s[16 * c2 + 4 * u + i] + dv[i] * pv[i];
          }
      }
    } else {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        v4f pv[4], dv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          pv[u] = mfma_k1_4(xu[u], w, zero4);
          if constexpr (MODE == 2) {
            v4i bits;
            for (int i = 0; i < 4; ++i) bits[i] = dacc[c2][4 * u + i];
            dv[u] = mfma_k1_4(-kMagic, 1.0f, __builtin_bit_cast(v4f, bits));
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if constexpr (MODE == 1)
            for (int i = 0; i < 4; ++i) dv[u][i] = (float)dacc[c2][4 * u + i];
          for (int i = 0; i < 4; ++i) s[16 * c2 + 4 * u + i] = s[16 * c2 + 4 * u + i] + dv[u][i] * pv[u][i];
        }
        asm volatile("" : "+v"(s));  // keep the rescale ahead of the next MFMAs
        __builtin_amdgcn_sched_barrier(0);
        const v16i c = MODE == 2 ? cinit : zero16i;
        dacc[c2] = c2 == 0 ? mfma_i8(a1, b01, mfma_i8(a0, b00, c)) : mfma_i8(a1, b11, mfma_i8(a0, b10, c));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float sum = 0;
  for (int i = 0; i < 32; ++i) sum += s[i];
  for (int i = 0; i < 16; ++i) sum += (float)dacc[0][i] + (float)dacc[1][i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
  const int gw = blockIdx.x * 4 + wid;
  if (lane == 0) {
    cyc[2 * gw] = t1 - t0;
    cyc[2 * gw + 1] = r1 - r0;
  }
}

typedef void (*Kernel)(int, long long*, float*);

void run(const char* name, Kernel k, int blocks_per_cu, int iters) {
  const int blocks = 256 * blocks_per_cu, waves = blocks * 4;
  long long* cyc;
  float* out;
  CHECK(hipMalloc(&cyc, sizeof(long long) * 2 * waves));
  CHECK(hipMalloc(&out, sizeof(float) * blocks * 256));
  k<<<blocks, 256>>>(10, cyc, out);
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  k<<<blocks, 256>>>(iters, cyc, out);
  CHECK(hipEventRecord(e1));
  CHECK(hipDeviceSynchronize());
  float ms;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<long long> h(2 * waves);
  CHECK(hipMemcpy(h.data(), cyc, sizeof(long long) * 2 * waves, hipMemcpyDeviceToHost));
  double c = 0, r = 0;
  for (int w = 0; w < waves; ++w) {
    c += h[2 * w];
    r += h[2 * w + 1];
  }
  const double ghz = c / (r * 10.0);  // s_memrealtime counts at 100 MHz
  const double simd_cyc = ms * 1e-3 * ghz * 1e9 / ((double)iters * blocks_per_cu);
  const double tops = 2.0 * 32 * 64 * 64 * (double)waves * iters / (ms * 1e-3) / 1e12;
  printf("%-40s waves/SIMD %d: %6.1f SIMD cycles per wave and group  clock %.2f GHz  %7.1f TOP/s (%.1f%% of 5.0 POPS)\n",
         name, blocks_per_cu, simd_cyc, ghz, tops, tops / 50.0);
  fflush(stdout);
  CHECK(hipFree(cyc));
  CHECK(hipFree(out));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  const int it = 3000;
  for (int b : {2, 3, 4}) {
    run("[0] kernel form (32x32x1 conv + prod)", k_inner<0>, b, it);
    run("[3] v_cvt conversion + 32x32x1 product", k_inner<3>, b, it);
    run("[4] 4x4x1 conversion + product", k_inner<4>, b, it);
    run("[1] pipelined, v_cvt + 4x4x1 product", k_inner<1>, b, it);
    run("[2] pipelined, 4x4x1 conversion + product", k_inner<2>, b, it);
  }
  return 0;
}

// Issue-rate microbenchmark for gfx950: how i8 MFMA, K=1 fp32 MFMA and plain
// fp32 VALU work share one SIMD.  The wide projection kernel's per-group work
// is exactly these three kinds (dots, conversion/product, t = dot * p and
// s = s + t), so their rates and overlap bound its speed.
//
// Every kernel runs a fixed loop on registers only (no memory traffic).  The
// host prints SIMD cycles per loop iteration from the wall time and the shader
// clock (s_memtime against the 100 MHz s_memrealtime).  Build and run:
//   make -C decider-engine_amd/microbench && decider-engine_amd/microbench/coexec
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#pragma clang fp contract(off)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e = (x);                                                       \
    if (e != hipSuccess) {                                                    \
      printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__);   \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

struct State {
  v4i a, b;
  v16i acc[4];
  v4f k1[16];
  float s[32], d[32], p[32];
  float ka, kb;
};

__device__ __forceinline__ void init(State& t, int lane) {
  t.a = v4i{lane, lane * 3, lane * 5, lane * 7};
  t.b = v4i{lane * 11, lane * 13, 1, 2};
  for (int j = 0; j < 4; ++j)
    for (int i = 0; i < 16; ++i) t.acc[j][i] = i + j;
  for (int j = 0; j < 16; ++j)
    for (int i = 0; i < 4; ++i) t.k1[j][i] = 0.0f;
  for (int i = 0; i < 32; ++i) {
    t.s[i] = 0.0f;
    t.d[i] = lane + i;
    t.p[i] = 1.0f / (i + 1);
  }
  t.ka = lane * 0.5f;
  t.kb = lane * 0.25f;
}

__device__ __forceinline__ float fold(State& t) {
  float sum = 0.0f;
  for (int j = 0; j < 4; ++j)
    for (int i = 0; i < 16; ++i) sum += (float)t.acc[j][i];
  for (int j = 0; j < 16; ++j)
    for (int i = 0; i < 4; ++i) sum += t.k1[j][i];
  for (int i = 0; i < 32; ++i) sum += t.s[i];
  return sum;
}

// One iteration: NI8 v_mfma_i32_32x32x32_i8, NK1 v_mfma_f32_4x4x1_16b_f32 and
// NV (v_mul_f32, v_add_f32) pairs, all independent.  IL interleaves them with
// sched_group_barrier (one MFMA, then its share of the VALU).
template <int NI8, int NK1, int NV, bool IL>
__device__ __forceinline__ void body(State& t) {
#pragma unroll
  for (int j = 0; j < NI8; ++j) t.acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(t.a, t.b, t.acc[j], 0, 0, 0);
#pragma unroll
  for (int j = 0; j < NK1; ++j) t.k1[j] = __builtin_amdgcn_mfma_f32_4x4x1f32(t.ka, t.kb, t.k1[j], 0, 0, 0);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    asm volatile("" : "+v"(t.d[i]));  // the operand changes every iteration
    const float x = t.d[i] * t.p[i];
    t.s[i] = t.s[i] + x;
  }
  if constexpr (IL) {
    constexpr int NM = NI8 + NK1;
    constexpr int per = NM > 0 ? (2 * NV) / NM : 0;
    constexpr int rem = NM > 0 ? 2 * NV - per * NM : 0;
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x8, 1, 0);    // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x2, per, 0);  // then VALU
    }
    if constexpr (rem > 0) __builtin_amdgcn_sched_group_barrier(0x2, rem, 0);
  }
}

template <int NI8, int NK1, int NV, bool IL>
__global__ __launch_bounds__(512) void k_mix(int iters, long long* cyc, float* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  State t;
  init(t, lane);
  const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) body<NI8, NK1, NV, IL>(t);
  const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  const int gw = blockIdx.x * (blockDim.x >> 6) + wid;
  out[blockIdx.x * blockDim.x + threadIdx.x] = fold(t);
  if (lane == 0) {
    cyc[2 * gw] = t1 - t0;
    cyc[2 * gw + 1] = r1 - r0;
  }
}

// Two kinds of waves on one SIMD: in 512-thread blocks waves w and w + 4 share
// a SIMD; waves with (w / 4) even run the MFMA body, the others the VALU body.
template <int AI8, int AK1, int BV>
__global__ __launch_bounds__(512) void k_split(int iters, long long* cyc, float* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  State t;
  init(t, lane);
  const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  if (((wid >> 2) & 1) == 0) {
    for (int it = 0; it < iters; ++it) body<AI8, AK1, 0, false>(t);
  } else {
    for (int it = 0; it < iters; ++it) body<0, 0, BV, false>(t);
  }
  const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  const int gw = blockIdx.x * (blockDim.x >> 6) + wid;
  out[blockIdx.x * blockDim.x + threadIdx.x] = fold(t);
  if (lane == 0) {
    cyc[2 * gw] = t1 - t0;
    cyc[2 * gw + 1] = r1 - r0;
  }
}

typedef void (*Kernel)(int, long long*, float*);

// blocks_per_cu blocks of `threads` on each of the 256 CUs; prints SIMD cycles
// per loop iteration of one wave (wall time x clock / iterations / waves per SIMD).
void run(const char* name, Kernel k, int blocks_per_cu, int threads, int iters) {
  const int blocks = 256 * blocks_per_cu;
  const int waves = blocks * threads / 64;
  long long* cyc;
  float* out;
  CHECK(hipMalloc(&cyc, sizeof(long long) * 2 * waves));
  CHECK(hipMalloc(&out, sizeof(float) * blocks * threads));
  k<<<blocks, threads>>>(10, cyc, out);
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  k<<<blocks, threads>>>(iters, cyc, out);
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
  const int wps = blocks_per_cu * threads / 256;
  const double simd_cyc = ms * 1e-3 * ghz * 1e9 / ((double)iters * wps);
  printf("%-36s waves/SIMD %d: %7.1f SIMD cycles per iteration  (clock %.2f GHz)\n", name, wps, simd_cyc, ghz);
  fflush(stdout);
  CHECK(hipFree(cyc));
  CHECK(hipFree(out));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  const int it = 4000;
  for (int b : {1, 2}) {
    run("4 i8 MFMA", k_mix<4, 0, 0, false>, b, 256, it);
    run("16 K=1 MFMA (4x4x1)", k_mix<0, 16, 0, false>, b, 256, it);
    run("64 VALU (32 mul + 32 add)", k_mix<0, 0, 32, false>, b, 256, it);
    run("4 i8 + 64 VALU, interleaved", k_mix<4, 0, 32, true>, b, 256, it);
    run("4 i8 + 16 K=1, interleaved", k_mix<4, 16, 0, true>, b, 256, it);
    run("4 i8 + 16 K=1 + 64 VALU, interleaved", k_mix<4, 16, 32, true>, b, 256, it);
    run("4 i8 + 16 K=1 + 64 VALU, in sequence", k_mix<4, 16, 32, false>, b, 256, it);
  }
  run("64 VALU (32 mul + 32 add)", k_mix<0, 0, 32, false>, 4, 256, it);
  run("split waves: 4 i8 | 64 VALU", k_split<4, 0, 32>, 1, 512, it);
  run("split waves: 4 i8 + 16 K=1 | 64 VALU", k_split<4, 16, 32>, 1, 512, it);
  run("split waves: 4 i8 | 64 VALU", k_split<4, 0, 32>, 2, 512, it);
  run("split waves: 4 i8 + 16 K=1 | 64 VALU", k_split<4, 16, 32>, 2, 512, it);
  return 0;
}

// Which MFMA kinds overlap plain fp32 VALU work on one gfx950 SIMD: i8
// 32x32x32 (the dots), f32 32x32x1_2b (the K=1 conversion and product of the
// wide kernel) and f16 32x32x16 (an exact alternative for the conversion:
// with every A and B element 768, the 16 products add 9437184 to a C that
// holds -(9437184 + dot) as a float, leaving -dot).  Every kernel runs a fixed
// loop on registers only; the host prints SIMD cycles per wave and iteration
// from the wall time and the shader clock (s_memtime against the 100 MHz
// s_memrealtime).  "il" interleaves the MFMAs with the VALU work
// (sched_group_barrier), "seq" issues them first.  Build and run:
//   make -C decider-engine_amd/microbench && decider-engine_amd/microbench/mfma_kinds
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#pragma clang fp contract(off)
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
#define CHECK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s line %d\n", hipGetErrorString(e), __LINE__); exit(1); } } while (0)

struct State {
  v4i a, b;
  v16i acc[2];
  v32f k1;
  v16f h[2];
  v8h ha, hb;
  float s[32], d[32];
  float ka, kb;
};
__device__ __forceinline__ void init(State& t, int lane) {
  t.a = v4i{lane, lane * 3, lane * 5, lane * 7};
  t.b = v4i{lane * 11, lane * 13, 1, 2};
  for (int j = 0; j < 2; ++j) for (int i = 0; i < 16; ++i) { t.acc[j][i] = i + j; t.h[j][i] = 0.0f; }
  for (int i = 0; i < 32; ++i) { t.k1[i] = 0.0f; t.s[i] = 0.0f; t.d[i] = lane + i; }
  for (int i = 0; i < 8; ++i) { t.ha[i] = (_Float16)(lane & 7); t.hb[i] = (_Float16)(i); }
  t.ka = lane * 0.5f; t.kb = lane * 0.25f;
}
template <int NI8, int NF32, int NF16, int NV>
__device__ __forceinline__ float fold(State& t) {
  float sum = 0.0f;
  if (NI8) for (int j = 0; j < 2; ++j) for (int i = 0; i < 16; ++i) sum += (float)t.acc[j][i];
  if (NF16) for (int j = 0; j < 1; ++j) for (int i = 0; i < 16; ++i) sum += t.h[j][i];
  if (NF32) for (int i = 0; i < 32; ++i) sum += t.k1[i];
  if (NV) for (int i = 0; i < 16; ++i) sum += t.s[i];
  return sum;
}
template <int NI8, int NF32, int NF16, int NV, bool IL>
__device__ __forceinline__ void body(State& t) {
#pragma unroll
  for (int j = 0; j < NI8; ++j) t.acc[j & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(t.a, t.b, t.acc[j & 1], 0, 0, 0);
#pragma unroll
  for (int j = 0; j < NF32; ++j) t.k1 = __builtin_amdgcn_mfma_f32_32x32x1f32(t.ka, t.kb, t.k1, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < NF16; ++j) t.h[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(t.ha, t.hb, t.h[0], 0, 0, 0);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    asm volatile("" : "+v"(t.d[i & 15]));
    const float x = t.d[i & 15] * t.d[(i + 1) & 15];
    t.s[i & 15] = t.s[i & 15] + x;
  }
  if constexpr (IL) {
    constexpr int NM = NI8 + NF32 + NF16;
    constexpr int per = NM > 0 ? (2 * NV) / NM : 0;
    constexpr int rem = NM > 0 ? 2 * NV - per * NM : 0;
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x8, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x2, per, 0);
    }
    if constexpr (rem > 0) __builtin_amdgcn_sched_group_barrier(0x2, rem, 0);
  }
}
template <int NI8, int NF32, int NF16, int NV, bool IL>
__global__ __launch_bounds__(512) void k_mix(int iters, long long* cyc, float* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  State t;
  init(t, lane);
  const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) body<NI8, NF32, NF16, NV, IL>(t);
  const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  const int gw = blockIdx.x * (blockDim.x >> 6) + wid;
  out[blockIdx.x * blockDim.x + threadIdx.x] = fold<NI8, NF32, NF16, NV>(t);
  if (lane == 0) { cyc[2 * gw] = t1 - t0; cyc[2 * gw + 1] = r1 - r0; }
}
typedef void (*Kernel)(int, long long*, float*);
void run(const char* name, Kernel k, int threads, int iters, int bpc = 1) {
  const int blocks = 256 * bpc, waves = blocks * threads / 64;
  long long* cyc; float* out;
  CHECK(hipMalloc(&cyc, sizeof(long long) * 2 * waves));
  CHECK(hipMalloc(&out, sizeof(float) * blocks * threads));
  k<<<blocks, threads>>>(10, cyc, out);
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1; CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  k<<<blocks, threads>>>(iters, cyc, out);
  CHECK(hipEventRecord(e1));
  CHECK(hipDeviceSynchronize());
  float ms; CHECK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<long long> h(2 * waves);
  CHECK(hipMemcpy(h.data(), cyc, sizeof(long long) * 2 * waves, hipMemcpyDeviceToHost));
  double c = 0, r = 0;
  for (int w = 0; w < waves; ++w) { c += h[2 * w]; r += h[2 * w + 1]; }
  const double ghz = c / (r * 10.0);
  const int wps = bpc * threads / 256;
  const double cycw = ms * 1e-3 * ghz * 1e9 / ((double)iters * wps);
  printf("%-44s waves/SIMD %d: %7.1f SIMD cycles per wave-iteration  (clock %.2f GHz)\n", name, wps, cycw, ghz);
  fflush(stdout);
  CHECK(hipFree(cyc)); CHECK(hipFree(out));
}
int main() {
  const int it = 4000;
  struct C { int th, bpc; };
  for (C c : {C{256, 1}, C{512, 1}, C{512, 2}}) {
    const int th = c.th, b = c.bpc;
    run("4 i8", k_mix<4, 0, 0, 0, false>, th, it, b);
    run("2 f32 32x32x1_2b", k_mix<0, 2, 0, 0, false>, th, it, b);
    run("2 f16 32x32x16", k_mix<0, 0, 2, 0, false>, th, it, b);
    run("64 VALU", k_mix<0, 0, 0, 32, false>, th, it, b);
    run("96 VALU", k_mix<0, 0, 0, 48, false>, th, it, b);
    run("4 i8 + 64 VALU, il", k_mix<4, 0, 0, 32, true>, th, it, b);
    run("2 f32 + 64 VALU, il", k_mix<0, 2, 0, 32, true>, th, it, b);
    run("2 f16 + 64 VALU, il", k_mix<0, 0, 2, 32, true>, th, it, b);
    run("4 i8 + 2 f32 + 64 VALU, il (kernel)", k_mix<4, 2, 0, 32, true>, th, it, b);
    run("4 i8 + 2 f32 + 64 VALU, seq (kernel)", k_mix<4, 2, 0, 32, false>, th, it, b);
    run("4 i8 + 2 f16 + 64 VALU, il", k_mix<4, 0, 2, 32, true>, th, it, b);
    run("4 i8 + 2 f16 + 96 VALU, il", k_mix<4, 0, 2, 48, true>, th, it, b);
    run("4 i8 + 2 f16 + 96 VALU, seq", k_mix<4, 0, 2, 48, false>, th, it, b);
    run("4 i8 + 128 VALU, il", k_mix<4, 0, 0, 64, true>, th, it, b);
    run("4 i8 + 1 f32 + 96 VALU, il", k_mix<4, 1, 0, 48, true>, th, it, b);
    run("4 i8 + 2 f16 + 1 f32 + 64 VALU, il", k_mix<4, 1, 2, 32, true>, th, it, b);
  }
  return 0;
}

// Issue-schedule microbenchmark for gfx950: the wide projection kernel's
// per-group arithmetic (4 i8 MFMA 32x32x32, the K=1 conversion and product
// MFMAs 32x32x1_2b, then t = dot * p and s = s + t on the VALU, 64
// instructions), with operands in registers or LDS, under three schedules:
//   seq : every wave runs its groups back to back (the shipped kernel's order);
//   pp  : blocks of 8 waves, two per SIMD; waves 0-3 and 4-7 alternate phases
//         through block barriers, so on every SIMD one wave issues its MFMA
//         phase while the other issues its VALU phase ("ping-pong");
//   bar : seq with one block barrier per group (the shipped kernel's sync).
// The host prints SIMD cycles per wave and group: wall time x shader clock /
// (groups x waves per SIMD).  Build and run:
//   make -C decider-engine_amd/microbench && decider-engine_amd/microbench/pingpong
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#pragma clang fp contract(off)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

#define CHECK(x)                                                            \
  do {                                                                      \
    hipError_t e = (x);                                                     \
    if (e != hipSuccess) {                                                  \
      printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__); \
      exit(1);                                                              \
    }                                                                       \
  } while (0)

constexpr int kMagicBits = 0x4B400000;
constexpr float kMagic = 12582912.0f;

__device__ __forceinline__ v32f concat(v16i lo, v16i hi) {
  v16f a = __builtin_bit_cast(v16f, lo), b = __builtin_bit_cast(v16f, hi);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20,
                                 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
}
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }
__device__ __forceinline__ void block_barrier() {
  sched_fence();
  __builtin_amdgcn_s_barrier();
  sched_fence();
}

enum { SEQ = 0, PP = 1, BAR = 2 };

// One wave and group.  MFMA phase: dots of a 32 x 64 tile (two 32x32 tiles,
// two K=32 steps each), then conversion and product.  VALU phase: 32 t's and
// 32 adds.  LDSR: the six 16-byte operand fragments come from LDS (distinct
// offsets per group, as the kernel's ring slots).
template <int MODE, bool LDSR>
__global__ __launch_bounds__(512) void k_group(int iters, long long* cyc, float* out) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][6][1024];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 2 * 6 * 1024 / 4; i += blockDim.x)
    reinterpret_cast<int*>(&lds[0][0][0])[i] = i * 2654435761u;
  __syncthreads();
  v4i a0 = v4i{lane, lane * 3, lane * 5, lane * 7}, a1 = a0 + 1;
  v4i b0 = v4i{lane * 11, lane * 13, 1, 2}, b1 = b0 + 2, b2 = b0 + 3, b3 = b0 + 4;
  v16i cinit;
  for (int i = 0; i < 16; ++i) cinit[i] = kMagicBits;
  v32f zero, s;
  for (int i = 0; i < 32; ++i) zero[i] = 0.0f, s[i] = 0.0f;
  float x = lane * 0.5f, w = lane * 0.25f;
  v32f dv, pv;
  const bool grp_b = wid >= 4;
  const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  if (MODE == PP && grp_b) block_barrier();
  for (int it = 0; it < iters; ++it) {
    if (LDSR) {
      const unsigned char* f = &lds[it & 1][0][0];
      a0 = *reinterpret_cast<const v4i*>(f + 16 * lane);
      a1 = *reinterpret_cast<const v4i*>(f + 1024 + 16 * lane);
      b0 = *reinterpret_cast<const v4i*>(f + 2048 + 16 * lane);
      b1 = *reinterpret_cast<const v4i*>(f + 3072 + 16 * lane);
      b2 = *reinterpret_cast<const v4i*>(f + 4096 + 16 * lane);
      b3 = *reinterpret_cast<const v4i*>(f + 5120 + 16 * lane);
    } else {
      asm volatile("" : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3));
    }
    asm volatile("" : "+v"(x), "+v"(w));
    v16i d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, cinit, 0, 0, 0);
    v16i d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b2, cinit, 0, 0, 0);
    d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, d0, 0, 0, 0);
    d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b3, d1, 0, 0, 0);
    dv = __builtin_amdgcn_mfma_f32_32x32x1f32(-kMagic, 1.0f, concat(d0, d1), 0, 0, 0);
    pv = __builtin_amdgcn_mfma_f32_32x32x1f32(x, w, zero, 0, 0, 0);
    if (MODE == PP) block_barrier();
    s = s + dv * pv;
    if (MODE != SEQ) block_barrier();
  }
  if (MODE == PP && !grp_b) block_barrier();
  const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float acc = 0.0f;
  for (int i = 0; i < 32; ++i) acc += s[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
  const int gw = blockIdx.x * (blockDim.x >> 6) + wid;
  if (lane == 0) {
    cyc[2 * gw] = t1 - t0;
    cyc[2 * gw + 1] = r1 - r0;
  }
}

typedef void (*Kernel)(int, long long*, float*);

// blocks_per_cu blocks of `threads` on each of the 256 CUs; prints SIMD cycles
// per wave and group.
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
  const double tops = 262144.0 * iters * waves / (ms * 1e-3) / 1e12;
  printf("%-44s waves/SIMD %d: %6.1f SIMD cycles per wave and group  clock %.2f GHz  %7.1f TOP/s (%.1f%%)\n", name,
         wps, simd_cyc, ghz, tops, tops / 50.0);
  fflush(stdout);
  CHECK(hipFree(cyc));
  CHECK(hipFree(out));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  const int it = 4000;
  run("seq, registers (8-wave blocks)", k_group<SEQ, false>, 1, 512, it);
  run("seq, LDS operands (8-wave blocks)", k_group<SEQ, true>, 1, 512, it);
  run("ping-pong, registers", k_group<PP, false>, 1, 512, it);
  run("ping-pong, LDS operands", k_group<PP, true>, 1, 512, it);
  run("barrier per group, registers (8-wave blocks)", k_group<BAR, false>, 1, 512, it);
  run("seq, LDS operands (4-wave blocks)", k_group<SEQ, true>, 4, 256, it);
  run("barrier per group, LDS (4-wave blocks)", k_group<BAR, true>, 4, 256, it);
  return 0;
}

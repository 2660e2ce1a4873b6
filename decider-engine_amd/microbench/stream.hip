// HBM streaming microbenchmark for gfx950: what one launch that only reads B
// bytes (16-byte loads, several in flight per lane) reaches, by launch size and
// wave count.  Launches rotate over 5 copies (5 x 73.6 MB > the 256 MB MALL),
// as the skinny projection workload does, so the bytes come from HBM.
// Reported per launch: HIP events around back-to-back launches on one stream
// (the host queues ahead of the GPU), averaged.  Build and run:
//   make -C decider-engine_amd/microbench && decider-engine_amd/microbench/stream
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                            \
  do {                                                                      \
    hipError_t e = (x);                                                     \
    if (e != hipSuccess) {                                                  \
      printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__); \
      exit(1);                                                              \
    }                                                                       \
  } while (0)

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Wave w reads 16-byte units [w*per, min((w+1)*per, units)) with its 64 lanes,
// D loads in flight per lane.  A lane stores its XOR only if it equals a value
// the data never gives, so nothing is written but no load can be dropped.
template <int D, bool NT>
__global__ __launch_bounds__(256) void k_stream(const v4u* __restrict__ src, long units, long per, unsigned* out) {
  const int lane = threadIdx.x & 63;
  const long wave = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long u0 = wave * per, u1 = u0 + per < units ? u0 + per : units;
  v4u acc = {0u, 0u, 0u, 0u};
  long u = u0 + lane;
  for (; u + 64 * (D - 1) < u1; u += 64 * D) {
    v4u v[D];
#pragma unroll
    for (int i = 0; i < D; ++i) v[i] = NT ? __builtin_nontemporal_load(src + u + 64 * i) : src[u + 64 * i];
#pragma unroll
    for (int i = 0; i < D; ++i) acc ^= v[i];
  }
  for (; u < u1; u += 64) acc ^= src[u];
  const unsigned r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9E3779B9u) out[wave & 1023] = r;
}

typedef void (*Kernel)(const v4u*, long, long, unsigned*);

int main() {
  const int copies = 5;
  const long max_bytes = 73601024;  // one question's weight bytes in the skinny workload
  std::vector<v4u*> buf(copies);
  for (int c = 0; c < copies; ++c) {
    CHECK(hipMalloc(&buf[c], max_bytes));
    CHECK(hipMemset(buf[c], c + 1, max_bytes));
  }
  unsigned* out;
  CHECK(hipMalloc(&out, 1024 * sizeof(unsigned)));
  CHECK(hipMemset(out, 0, 1024 * sizeof(unsigned)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  struct Case {
    long bytes;
    int waves;
    int depth;
    bool nt;
  };
  // The skinny launches' shapes: 17.9 MB over 260 waves (one projection's 32-column strips), 60.2 MB over 868
  // waves (eight projections' strips), 12 loads in flight per lane as their register rings hold.
  const Case cases[] = {
      {73601024, 1024, 4, true},  {73601024, 1536, 4, true},  {73601024, 2048, 4, true},
      {73601024, 4096, 4, true},  {73601024, 8192, 4, true},  {73601024, 2048, 8, true},
      {73601024, 4096, 8, true},  {73601024, 1024, 4, false}, {73601024, 2048, 4, false},
      {73601024, 4096, 4, false}, {16777216, 2048, 4, true},  {16777216, 4096, 4, true},
      {16777216, 8192, 2, true},  {16777216, 4096, 4, false}, {17907712, 260, 4, false},
      {17907712, 260, 12, false}, {17907712, 1040, 4, false}, {17907712, 1040, 12, false},
      {60162048, 868, 4, false},  {60162048, 868, 12, false}, {60162048, 3472, 4, false},
  };
  for (const Case& cs : cases) {
    const long units = cs.bytes / 16;
    const long per = (units + cs.waves - 1) / cs.waves;
    const int blocks = (cs.waves + 3) / 4;
    Kernel k = cs.nt ? (cs.depth == 8 ? k_stream<8, true> : cs.depth == 2 ? k_stream<2, true> : k_stream<4, true>)
                     : (cs.depth == 8 ? k_stream<8, false> : cs.depth == 12 ? k_stream<12, false>
                                                           : cs.depth == 2 ? k_stream<2, false> : k_stream<4, false>);
    for (int i = 0; i < copies; ++i) k<<<blocks, 256>>>(buf[i], units, per, out);
    CHECK(hipDeviceSynchronize());
    const int reps = 50;
    CHECK(hipEventRecord(e0));
    for (int i = 0; i < reps; ++i) k<<<blocks, 256>>>(buf[i % copies], units, per, out);
    CHECK(hipEventRecord(e1));
    CHECK(hipDeviceSynchronize());
    float ms;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double us = ms * 1e3 / reps;
    printf("read %6.1f MB  waves %5d  loads in flight per lane %d  %s: %6.2f us per launch  %6.0f GB/s (%.1f%% of 8 TB/s)\n",
           cs.bytes / 1e6, cs.waves, cs.depth, cs.nt ? "non-temporal" : "plain       ", us, cs.bytes / (us * 1e-6) / 1e9, cs.bytes / (us * 1e-6) / 8e12 * 100);
    fflush(stdout);
  }
  for (int c = 0; c < copies; ++c) CHECK(hipFree(buf[c]));
  CHECK(hipFree(out));
  return 0;
}

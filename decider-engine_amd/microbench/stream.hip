// HBM streaming microbenchmark for gfx950: what one launch that only reads B
// bytes (16-byte loads, several in flight per lane) reaches, by launch size and
// wave count.  Launches rotate over 5 copies (5 x 73.6 MB > the 256 MB MALL),
// as the skinny projection workload does, so the bytes come from HBM.
// Reported per launch: HIP events around back-to-back launches on one stream
// (the host queues ahead of the GPU), averaged.  A second part streams the
// skinny question launch's own distribution of weight bytes over waves.
// Build and run:
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

// Wave w reads units [off[w], off[w] + cnt[w]) of src (16 B each), 4 loads in
// flight per lane: the skinny launch's distribution of weight bytes over waves.
__global__ __launch_bounds__(256) void k_list(const v4u* __restrict__ src, const long* __restrict__ off,
                                              const int* __restrict__ cnt, int waves, unsigned* out) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= waves) return;
  const long u0 = off[w], u1 = u0 + cnt[w];
  v4u acc = {0u, 0u, 0u, 0u};
  long u = u0 + lane;
  for (; u + 64 * 3 < u1; u += 64 * 4) {
    v4u v0 = src[u], v1 = src[u + 64], v2 = src[u + 128], v3 = src[u + 192];
    acc ^= v0; acc ^= v1; acc ^= v2; acc ^= v3;
  }
  for (; u < u1; u += 64) acc ^= src[u];
  const unsigned r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9E3779B9u) out[w & 1023] = r;
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
  // The skinny question launch's own distribution (73.6 MB per launch: down, K = 6144, 128 strips of 16 columns
  // read by two 4-wave blocks each, first; then the eight short-K projections as 868 strips of 32 columns, one per
  // wave, 4 per block), against balanced distributions of the same bytes.
  {
    const long bytes = 73601024, units = bytes / 16;
  struct Case { const char* name; std::vector<long> off; std::vector<int> cnt; };
    std::vector<Case> cases;
    const long downB = 12582912 + 2048 * 96 * 4;  // down weights + scales
    const long shortB = bytes - downB;             // the other eight projections
    auto add_down = [&](Case& c, bool dup) {
      // 128 strips of 16 columns x 6144; 2 blocks per strip (row tiles), 4 waves per block, each wave 1/4 of the strip
      const long strip = downB / 128 / 16;  // units per strip
      for (int s = 0; s < 128; ++s)
        for (int t = 0; t < (dup ? 2 : 1); ++t)
          for (int w = 0; w < 4; ++w) { c.off.push_back(shortB / 16 + s * strip + w * (strip / 4)); c.cnt.push_back((int)(strip / 4)); }
    };
    auto add_short = [&](Case& c, long nstrips, int per_wave_strips) {
      const long strip = shortB / 16 / nstrips;  // units per strip
      long s = 0;
      while (s < nstrips) {
        for (int w = 0; w < 4; ++w) {
          const long a = s, b = std::min(nstrips, s + per_wave_strips);
          c.off.push_back(a * strip); c.cnt.push_back((int)((b - a) * strip));
          s = b;
        }
      }
    };
    { Case c{"skinny-like: 256 down blocks (2 per strip) then 217 short blocks of 4 x 64 KB"}; add_down(c, true); add_short(c, 868, 1); cases.push_back(c); }
    { Case c{"down once (128 blocks) then 217 short blocks"}; add_down(c, false); add_short(c, 868, 1); cases.push_back(c); }
    { Case c{"256 down blocks then 256 short blocks (balanced bytes)"}; add_down(c, true);
      const long per = shortB / 16 / 1024; for (int w = 0; w < 1024; ++w) { c.off.push_back(w * per); c.cnt.push_back((int)per); } cases.push_back(c); }
    { Case c{"short only: 217 blocks of 4 x 64 KB"}; add_short(c, 868, 1); cases.push_back(c); }
    { Case c{"short only: 256 blocks balanced"}; const long per = shortB / 16 / 1024; for (int w = 0; w < 1024; ++w) { c.off.push_back(w * per); c.cnt.push_back((int)per); } cases.push_back(c); }
    { Case c{"all bytes over 1024 waves, balanced"}; const long per = units / 1024; for (int w = 0; w < 1024; ++w) { c.off.push_back(w * per); c.cnt.push_back((int)per); } cases.push_back(c); }
    { Case c{"all bytes over 2048 waves, balanced"}; const long per = units / 2048; for (int w = 0; w < 2048; ++w) { c.off.push_back(w * per); c.cnt.push_back((int)per); } cases.push_back(c); }
    for (auto& c : cases) {
      const int waves = (int)c.off.size();
      long maxu = 0;
      for (int w = 0; w < waves; ++w) maxu = std::max(maxu, c.off[w] + c.cnt[w]);
      if (maxu > units) { printf("bad case %s\n", c.name); continue; }
      long* doff; int* dcnt;
      CHECK(hipMalloc(&doff, waves * sizeof(long))); CHECK(hipMalloc(&dcnt, waves * sizeof(int)));
      CHECK(hipMemcpy(doff, c.off.data(), waves * sizeof(long), hipMemcpyHostToDevice));
      CHECK(hipMemcpy(dcnt, c.cnt.data(), waves * sizeof(int), hipMemcpyHostToDevice));
      const int blocks = (waves + 3) / 4;
      for (int i = 0; i < copies; ++i) k_list<<<blocks, 256>>>(buf[i], doff, dcnt, waves, out);
      CHECK(hipDeviceSynchronize());
      const int reps = 50;
      CHECK(hipEventRecord(e0));
      for (int i = 0; i < reps; ++i) k_list<<<blocks, 256>>>(buf[i % copies], doff, dcnt, waves, out);
      CHECK(hipEventRecord(e1));
      CHECK(hipDeviceSynchronize());
      float ms; CHECK(hipEventElapsedTime(&ms, e0, e1));
      long tot = 0; for (int w = 0; w < waves; ++w) tot += c.cnt[w];
      const double us = ms * 1e3 / reps;
      printf("%-80s waves %5d  %6.1f MB read  %6.2f us  %6.0f GB/s of 73.6 MB\n", c.name, waves, tot * 16 / 1e6, us, bytes / (us * 1e-6) / 1e9);
      fflush(stdout);
      CHECK(hipFree(doff)); CHECK(hipFree(dcnt));
    }
  }
  for (int c = 0; c < copies; ++c) CHECK(hipFree(buf[c]));
  CHECK(hipFree(out));
  return 0;
}

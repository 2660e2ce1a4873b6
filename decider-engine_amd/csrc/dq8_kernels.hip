// HIP kernels for gfx950 (CDNA4): group-64 int8 quantization, weight repack and
// the bit-exact int8 projection.
//
// Arithmetic contract (decider-engine src/int8.rs:53-61, src/tensor.rs:427-437):
// for every output (m, n), s = +0.0f and for each group g in order
//     p = xs[m][g] * ws[n][g];  t = (float)dot_g * p;  s = s + t
// with three separately rounded fp32 operations, then y = s + bias (0.0 if none).
//
// Mapping onto CDNA4:
//  * dot_g comes from v_mfma_i32_32x32x32_i8 (two per group, chained through C).
//    C starts at 0x4B400000 (the bits of 1.5*2^23), so the i32 result is
//    0x4B400000 + dot_g; since |dot_g| <= 2^20 those bits are the float
//    12582912 + dot_g exactly.
//  * v_mfma_f32_32x32x1_2b_f32 with A = -12582912, B = 1 and C = those bits
//    returns dot_g as an exact float for two 32x32 tiles (conversion off the VALU).
//  * The same K=1 instruction with A = x scales and B = w scales and C = 0 is an
//    outer product: p for two 32x32 tiles, each element one correctly rounded
//    product (its output layout equals the i8 tile layout).
//  * t and s are plain v_mul_f32 / v_add_f32 (contraction disabled).
#include "dq8_internal.h"

#include <float.h>
#include <math.h>

#pragma clang fp contract(off)

namespace dq8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kMagicBits = 0x4B400000;
constexpr float kMagic = 12582912.0f;

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v32f mfma_k1(float a, float b, v32f c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v32f concat(v16i lo, v16i hi) {
  v16f a = __builtin_bit_cast(v16f, lo), b = __builtin_bit_cast(v16f, hi);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20,
                                 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
}
__device__ __forceinline__ v4i load16(const void* p) { return *reinterpret_cast<const v4i*>(p); }

// silu (decider-engine src/qwen.rs:194-199): x * (1 / (1 + exp(-x))).
// exp is evaluated in double and rounded once to float.
__device__ __forceinline__ float silu(float x) {
  float e = (float)exp(-(double)x);
  return x * (1.0f / (1.0f + e));
}

// Epilogue::store (tensor.rs:92-99) through write_columns (tensor.rs:272-288)
// for E values of one lane at (row[e], col[e]); elements outside m x n are
// skipped.  Layout and epilogue are uniform, so they are branched on once, and
// every old value an Add/SwiGlu store reads is loaded before the first store.
template <int E>
__device__ __forceinline__ void store_tile(const Proj& P, const int (&row)[E], const int (&col)[E],
                                           const float (&y)[E]) {
  if (P.layout == 1) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (row[e] < P.m && col[e] < P.n) P.out[(size_t)col[e] * P.m + row[e]] = y[e];
    return;
  }
  if (P.epilogue == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (row[e] < P.m && col[e] < P.n) P.out[(size_t)row[e] * P.n + col[e]] = y[e];
    return;
  }
  float old[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    old[e] = row[e] < P.m && col[e] < P.n ? P.out[(size_t)row[e] * P.n + col[e]] : 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (row[e] < P.m && col[e] < P.n)
      P.out[(size_t)row[e] * P.n + col[e]] = P.epilogue == 1 ? old[e] + y[e] : silu(old[e]) * y[e];
}

__device__ __forceinline__ int find_proj(const Batch& b, int wave) {
  int pi = 0;
  for (int i = 1; i < b.count; ++i)
    if (wave >= b.p[i].wave_begin) pi = i;
  return pi;
}

// ---------------------------------------------------------------------------
// Quantization: QuantizedInputs::new (tensor.rs:321-339) and the 8-bit
// Data::quantize (weights.rs:117-136).  One wave covers 256 consecutive
// elements of a row (4 per lane, 4 groups per wave); a group's absmax is a
// max-reduction over its 16 lanes.  The division is the IEEE one and roundf
// rounds half away from zero, as f32::round.
__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ x, int rows, int k, int8_t* __restrict__ q,
                                                  int ldq, float* __restrict__ scales, uint32_t* nonfinite) {
  const int lane = threadIdx.x & 63;
  const int chunks = (k + 255) >> 8;
  const long item = (long)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  if (item >= (long)rows * chunks) return;
  const int row = (int)(item / chunks);
  const int chunk = (int)(item - (long)row * chunks);
  const int k0 = chunk * 256 + lane * 4;
  const float* xr = x + (size_t)row * k;
  float v[4];
  if ((k & 3) == 0 && k0 + 3 < k && ((uintptr_t)x & 15) == 0) {
    float4 t = *reinterpret_cast<const float4*>(xr + k0);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (k0 + i < k) ? xr[k0 + i] : 0.0f;
  }
  bool bad = false;
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bad |= !isfinite(v[i]);
    m = fmaxf(m, fabsf(v[i]));
  }
  if (bad && nonfinite) atomicOr(nonfinite, 1u);
  // max over the 16 lanes of this group (fmaxf of non-negative values is order-free)
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  m = fmaxf(m, __shfl_xor(m, 4));
  m = fmaxf(m, __shfl_xor(m, 8));
  const float scale = (m == 0.0f) ? 1.0f : fmaxf(m / 127.0f, FLT_MIN);
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float r = roundf(v[i] / scale);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    packed |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * i);
  }
  int8_t* qr = q + (size_t)row * ldq;
  if ((ldq & 3) == 0 && k0 + 3 < ldq && ((uintptr_t)q & 3) == 0) {
    // Padding bytes [k, ldq) are written as zero (v = 0 there).
    *reinterpret_cast<uint32_t*>(qr + k0) = packed;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (k0 + i < ldq) qr[k0 + i] = (int8_t)(packed >> (8 * i));
  }
  const int group = (chunk * 256 + (lane & ~15) * 4) / kGroup;
  const int groups = (k + kGroup - 1) / kGroup;
  if ((lane & 15) == 0 && group < groups) scales[(size_t)row * groups + group] = scale;
}

// Reference layout -> fragment layout (see Weights in dq8_internal.h).
__global__ void k_repack_values(const uint8_t* __restrict__ values, int n, int k, int g, uint8_t* __restrict__ wt,
                                long chunks) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= chunks) return;
  const int lane = (int)(i & 63);
  const int h = (int)((i >> 6) & 1);
  const long rest = i >> 7;
  const int gi = (int)(rest % g);
  const int nb = (int)(rest / g);
  const int row = nb * 32 + (lane & 31);
  const int k0 = gi * kGroup + 32 * h + 16 * (lane >> 5);
  uint32_t w[4] = {0, 0, 0, 0};
  if (row < n) {
    const uint8_t* src = values + (size_t)row * k;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (k0 + j < k) w[j >> 2] |= (uint32_t)src[k0 + j] << (8 * (j & 3));
  }
  *reinterpret_cast<uint4*>(wt + i * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

// wst has G + 1 rows; row G is all zero (the scale of groups past the end).
__global__ void k_repack_scales(const float* __restrict__ scales, int n, int g, int np, float* __restrict__ wst) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)(g + 1) * np) return;
  const int gi = (int)(i / np), col = (int)(i % np);
  wst[i] = (col < n && gi < g) ? scales[(size_t)col * g + gi] : 0.0f;
}

__global__ void k_export_values(const uint8_t* __restrict__ wt, int n, int k, int g, uint8_t* __restrict__ values) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)n * k) return;
  const int row = (int)(i / k), kk = (int)(i % k);
  const int nb = row >> 5, gi = kk / kGroup, h = (kk % kGroup) / 32;
  const int lane = (row & 31) + 32 * ((kk & 31) >> 4);
  values[i] = wt[((((long)nb * g + gi) * 2 + h) * 64 + lane) * 16 + (kk & 15)];
}

__global__ void k_export_scales(const float* __restrict__ wst, int n, int g, int np, float* __restrict__ scales) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)n * g) return;
  const int row = (int)(i / g), gi = (int)(i % g);
  scales[i] = wst[(size_t)gi * np + row];
}

// Copy q [rows][k] into dst [rows][ldq] with zero padding (ldq = G*64).
__global__ void k_pad_rows(const int8_t* __restrict__ q, int rows, int k, int8_t* __restrict__ dst, int ldq) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * ldq) return;
  const int row = (int)(i / ldq), kk = (int)(i % ldq);
  dst[i] = kk < k ? q[(size_t)row * k + kk] : (int8_t)0;
}

// ---------------------------------------------------------------------------
// Wide projection kernel (M > 32), LDS-staged.  A block of WM x WN waves owns
// a (64*WM) x (64*WN) output tile; each wave owns 64 x 64 of it: row tiles
// r0, r1 (32 rows each) x column tiles j0, j1.  Per group, for each column
// tile j the pair (r0, j), (r1, j) shares one conversion MFMA and one product
// MFMA: A lane l carries the x scale of row m0 + l, B lane l the w scale of
// column n0 + 32j + l%32.
//
// Operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4:
// lane l's 16 bytes land at base + 16*l, i.e. fragments stay in lane order and
// LDS reads are conflict-free ds_read_b128).  STAGES groups are in flight in
// an LDS ring.  Iteration g: wait for this wave's loads of group g
// (vmcnt <= loads of the STAGES-2 newer groups), barrier (every wave's loads
// of group g have landed and every wave is done reading group g-1), issue the
// loads of group g+STAGES-1 into group g-1's buffer, then read group g and
// compute.  Groups past the end load clamped operands and the all-zero w scale
// row G, so p = 0, t = dot * 0 = +-0 and s + t = s (s is never -0).

// Tile (row tile mt, column tile nt) of block i of a projection.  Blocks are
// dealt to the 8 XCDs round robin, so blocks i, i+8, ... share one XCD and its
// L2.  With P.xcd_gm = gm the tile grid is cut into gm x (8/gm) regions and
// XCD i%8 walks region i%8, column tiles fastest: it touches 1/gm of the
// activation rows and 1/(8/gm) of the weight columns.  The map is a bijection
// on [0, row_tiles * col_tiles) (the host picks gm dividing both counts).
__device__ __forceinline__ void tile_of(const Proj& P, int i, int row_tiles, int& mt, int& nt) {
  const int col_tiles = P.waves_n;
  if (P.xcd_gm == 0) {
    mt = i / col_tiles;
    nt = i - mt * col_tiles;
    return;
  }
  const int gm = P.xcd_gm, gn = 8 / gm;
  const int rm = row_tiles / gm, rn = col_tiles / gn;  // region size in tiles
  const int x = i & 7, j = i >> 3;
  const int xa = x / gn, xb = x - xa * gn;
  const int lm = j / rn;
  mt = xa * rm + lm;
  nt = xb * rn + (j - lm * rn);
}

// Direct global->LDS loads.  They are issued through inline assembly so the
// compiler does not track them: its LDS-DMA bookkeeping is conservative at
// loop headers and would drain the whole pipeline there.  The kernel orders
// every use itself (wait_vmcnt + s_barrier).  No compiler-generated code in
// these kernels uses M0; the s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma16(const void* src, const void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_offset(lds)), "v"(src)
               : "memory");
}
__device__ __forceinline__ void dma4(const void* src, const void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds_offset(lds)), "v"(src)
               : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Launch shape of the wide kernel (tunable at build time):
//   WM x WN waves per block, each wave (32*RT) rows x (32*CT) columns;
//   STAGES groups in flight in LDS; CVT_VALU converts the dots on the VALU
//   (C = 0) instead of the K=1 MFMA (C = bias bits).
#ifndef DQ8_WIDE_WM
#define DQ8_WIDE_WM 2
#endif
#ifndef DQ8_WIDE_WN
#define DQ8_WIDE_WN 2
#endif
#ifndef DQ8_WIDE_RT
#define DQ8_WIDE_RT 1
#endif
#ifndef DQ8_WIDE_CT
#define DQ8_WIDE_CT 2
#endif
#ifndef DQ8_WIDE_STAGES
#define DQ8_WIDE_STAGES 4
#endif
#ifndef DQ8_WIDE_CVT_VALU
#define DQ8_WIDE_CVT_VALU 0
#endif

// A wave's 32x32 tiles are processed in pairs that share one conversion and one
// product MFMA (blocks 0 and 1 of v_mfma_f32_32x32x1_2b_f32):
//   RT == 2: pair j = row tiles (0, 1) at column tile j;  A lane l: x of row l,
//            B lane l: w of column 32j + l%32.
//   RT == 1: one pair = column tiles (0, 1) at the single row tile;  A lane l:
//            x of row l%32, B lane l: w of column l.
template <int WM, int WN, int RT, int CT, int STAGES, bool CVT_VALU, bool DOTS>
__global__ __launch_bounds__(64 * WM * WN) void k_linear_wide(Batch b) {
  constexpr int NW = WM * WN, WR = 32 * RT, WC = 32 * CT;  // wave tile WR x WC
  constexpr int BM = WR * WM, BN = WC * WN;
  constexpr int AF = BM / 16, BF = BN / 16, NF = AF + BF;  // 1 KB fragments per group
  constexpr int FPW = NF / NW;
  constexpr int SCW = (BM + BN) / 64;           // waves holding real scales
  constexpr int LOADS = FPW + (DOTS ? 0 : 1);   // DMA instructions per wave per group
  constexpr int NP = RT == 2 ? CT : 1;          // pairs per wave
  static_assert(NF % NW == 0, "fragments must split evenly over the waves");
  static_assert(BM % 64 == 0 && BN % 64 == 0 && SCW <= NW, "64 scales per staging wave");
  static_assert((RT == 2 && (CT == 1 || CT == 2)) || (RT == 1 && CT == 2), "supported wave tiles");
  static_assert(STAGES >= 2 && STAGES <= 4 && LOADS * (STAGES - 2) <= 63, "pipeline depth");
  // One LDS object per stage, always indexed by compile-time constants.
  struct Stage {
    uint8_t frag[NF][kFragBytes];
    float sc[64 * NW];  // x scales of the BM rows, w scales of the BN columns, then padding
  };
  __shared__ __attribute__((aligned(16))) Stage st0, st1, st2, st3;
  auto stage = [&](int i) -> Stage& { return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3; };

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int blk = blockIdx.x;
  const Proj P = b.p[find_proj(b, blk)];  // by value: fields stay in registers across the stores
  int mt, nt;
  tile_of(P, blk - P.wave_begin, (P.m + BM - 1) / BM, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int G = P.g;

  // Global sources of this wave's fragments: A (row tile, half) or B (column tile, half).
  const uint8_t* src[FPW];
  int stride[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = wid + i * NW;
    if (f < AF) {
      const int row = min(m0 + 32 * (f >> 1) + (lane & 31), P.m - 1);
      src[i] = reinterpret_cast<const uint8_t*>(P.q) + (size_t)row * P.ldq + 32 * (f & 1) + 16 * (lane >> 5);
      stride[i] = kGroup;
    } else {
      const int fb = f - AF;
      src[i] = P.wt + ((size_t)(n0 / 32 + (fb >> 1)) * G * 2 + (fb & 1)) * kFragBytes + lane * 16;
      stride[i] = 2 * kFragBytes;
    }
  }
  // Scales: the first BM/64 waves stage x scales of 64 rows each, the next BN/64
  // waves w scales of 64 columns; the rest load a harmless duplicate into the
  // padding so that every wave issues the same number of loads.  x scales clamp
  // to the last group, w scales run into the zero row G.
  const int sw = wid < SCW ? wid : 0;
  const bool xwave = sw < BM / 64;
  const float* psc = xwave ? P.xs + (size_t)min(m0 + 64 * sw + lane, P.m - 1) * G
                           : P.wst + n0 + 64 * (sw - BM / 64) + lane;
  const size_t sstride = xwave ? 1 : (size_t)P.np;
  const int slast = xwave ? G - 1 : G;

  auto issue = [&](Stage& S, int g) {
    const int gc = min(g, G - 1);
#pragma unroll
    for (int i = 0; i < FPW; ++i) dma16(src[i] + (size_t)gc * stride[i], &S.frag[wid + i * NW][0]);
    if constexpr (!DOTS) dma4(psc + (size_t)min(g, slast) * sstride, &S.sc[64 * wid]);
  };

  const int wm = wid / WN, wn = wid - (wid / WN) * WN;
  const int fa = 2 * RT * wm;   // first A fragment of this wave
  const int fbw = AF + 2 * CT * wn;  // first B fragment

  v16i cinit;
#pragma unroll
  for (int i = 0; i < 16; ++i) cinit[i] = CVT_VALU ? 0 : kMagicBits;
  v32f zero32;
#pragma unroll
  for (int i = 0; i < 32; ++i) zero32[i] = 0.0f;
  v32f s[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) s[j] = zero32;

#pragma unroll
  for (int i = 0; i < STAGES - 1; ++i) {
    issue(stage(i), i);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int g0 = 0; g0 < G; g0 += STAGES) {
#pragma unroll
    for (int d = 0; d < STAGES; ++d) {
      const int g = g0 + d;
      if (g >= G) break;  // uniform over the block
      Stage& cur = stage(d);
      wait_vmcnt<LOADS * (STAGES - 2)>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue(stage((d + STAGES - 1) % STAGES), g + STAGES - 1);
      __builtin_amdgcn_sched_barrier(0);
      const v4i* fr = reinterpret_cast<const v4i*>(&cur.frag[0][0]);
      v4i af[RT][2], bf[CT][2];
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        af[r][0] = fr[(fa + 2 * r) * 64 + lane];
        af[r][1] = fr[(fa + 2 * r + 1) * 64 + lane];
      }
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        bf[j][0] = fr[(fbw + 2 * j) * 64 + lane];
        bf[j][1] = fr[(fbw + 2 * j + 1) * 64 + lane];
      }
      // dt[r][j]: dot tile of row tile r, column tile j (two MFMAs, K = 32 each).
      v16i dt[RT][CT];
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int j = 0; j < CT; ++j) dt[r][j] = mfma_i8(af[r][0], bf[j][0], cinit);
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int j = 0; j < CT; ++j) dt[r][j] = mfma_i8(af[r][1], bf[j][1], dt[r][j]);
      if constexpr (DOTS) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
          for (int j = 0; j < CT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int row = m0 + WR * wm + 32 * r + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
              const int col = n0 + WC * wn + 32 * j + (lane & 31);
              if (row < P.m && col < P.n)
                P.dots[((size_t)row * P.n + col) * G + g] = dt[r][j][v] - (CVT_VALU ? 0 : kMagicBits);
            }
      } else {
#pragma unroll
        for (int j = 0; j < NP; ++j) {
          const v16i& lo = RT == 2 ? dt[0][j] : dt[0][0];
          const v16i& hi = RT == 2 ? dt[1][j] : dt[0][1];
          float x, w;
          if constexpr (RT == 2) {
            x = cur.sc[WR * wm + lane];
            w = cur.sc[BM + WC * wn + 32 * j + (lane & 31)];
          } else {
            x = cur.sc[WR * wm + (lane & 31)];
            w = cur.sc[BM + WC * wn + lane];
          }
          v32f dv;
          if constexpr (CVT_VALU) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              dv[v] = (float)lo[v];
              dv[16 + v] = (float)hi[v];
            }
          } else {
            dv = mfma_k1(-kMagic, 1.0f, concat(lo, hi));
          }
          const v32f pv = mfma_k1(x, w, zero32);
          s[j] = s[j] + dv * pv;
        }
      }
    }
  }
  // Drain the clamped loads of the groups past the end before the block exits.
  wait_vmcnt<0>();
  if constexpr (!DOTS) {
    const int mw = m0 + WR * wm, nw = n0 + WC * wn;
    // y = s + bias[col], or s + 0.0f without a bias (tensor.rs:437)
    float bias[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int col = nw + 32 * c + (lane & 31);
      bias[c] = P.bias != nullptr && col < P.n ? P.bias[col] : 0.0f;
    }
    constexpr int E = NP * 32;
    int rows[E], cols[E];
    float y[E];
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int v = 0; v < 32; ++v) {
        const int blk2 = v >> 4, vv = v & 15;
        const int r = RT == 2 ? blk2 : 0, c = RT == 2 ? j : blk2;
        rows[32 * j + v] = mw + 32 * r + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);
        cols[32 * j + v] = nw + 32 * c + (lane & 31);
        y[32 * j + v] = s[j][v] + bias[c];
      }
    store_tile(P, rows, cols, y);
  }
}

// ---------------------------------------------------------------------------
// Skinny projection kernel, 16 x 16 wave tiles (M <= 32).  Each wave owns one
// 16-row tile x 16 columns and walks the groups one at a time:
//   v_mfma_i32_16x16x64_i8 gives one group's dots for the tile (row
//   4*(l/16) + v, column l%16), C = the bias bits 0x4B400000;
//   v_mfma_f32_4x4x1_16b_f32 with A = -12582912, B = 1 converts them exactly;
//   the same instruction with A lane a = x of row 4*(a/16) + a%4 and B lane l =
//   w of column l%16 is the product outer product in the same layout.
// The row tiles of one 16-column strip are adjacent waves of a block, so the
// strip's weights come from HBM once and from L1/L2 for the other row tiles.
// Short dependency chains and many waves hide the memory latency.
struct Skinny16Frag {
  v4i a, b;
  float x, w;
};

__device__ __forceinline__ v4i mfma_i8_16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_k1_4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

template <int DEPTH, bool DOTS>
__global__ __launch_bounds__(256) void k_linear_skinny16(Batch b) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave >= b.total_waves) return;
  const Proj P = b.p[find_proj(b, wave)];
  const int rtiles = (P.m + 15) >> 4;
  const int w_local = wave - P.wave_begin;
  const int nt = w_local / rtiles;  // 16-column strip
  const int r0 = (w_local - nt * rtiles) * 16;
  const int c0 = nt * 16;
  const int G = P.g;

  // A: lane l holds row r0 + l%16, bytes 16*(l/16) of the group.
  const int8_t* pa = P.q + (size_t)min(r0 + (lane & 15), P.m - 1) * P.ldq + 16 * (lane >> 4);
  const float* pxs = P.xs + (size_t)min(r0 + 4 * (lane >> 4) + (lane & 3), P.m - 1) * G;  // K=1 A-lane row
  // B: lane l holds column c0 + l%16, bytes 16*(l/16): in the 32-row fragment
  // layout that is half l/32, lane (c0%32) + l%16 + 32*((l/16)&1).
  const uint8_t* pb = P.wt + ((size_t)(c0 / 32) * G * 2 + (lane >> 5)) * kFragBytes +
                      ((c0 & 31) + (lane & 15) + 32 * ((lane >> 4) & 1)) * 16;
  const float* pws = P.wst + c0 + (lane & 15);

  auto load = [&](Skinny16Frag& f, int g) {
    const int gc = min(g, G - 1);
    f.a = load16(pa + gc * kGroup);
    f.b = load16(pb + (size_t)gc * 2 * kFragBytes);
    if constexpr (!DOTS) {
      f.x = pxs[gc];
      f.w = pws[(size_t)min(g, G) * P.np];  // row G of the w scales is zero
    }
  };

  v4i magic = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  v4f s = zero4;

  Skinny16Frag ring[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    load(ring[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int g0 = 0; g0 < G; g0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int g = g0 + d;
      const Skinny16Frag& c = ring[d];
      const v4i dd = mfma_i8_16(c.a, c.b, magic);
      v4f pv;
      if constexpr (!DOTS) pv = mfma_k1_4(c.x, c.w, zero4);
      // Refill the slot once every operand of it is consumed.
      __builtin_amdgcn_sched_barrier(0);
      load(ring[d], g + DEPTH);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DOTS) {
        if (g < G) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = r0 + 4 * (lane >> 4) + v;
            const int col = c0 + (lane & 15);
            if (row < P.m && col < P.n) P.dots[((size_t)row * P.n + col) * G + g] = dd[v] - kMagicBits;
          }
        }
      } else {
        const v4f dv = mfma_k1_4(-kMagic, 1.0f, __builtin_bit_cast(v4f, dd));
        s = s + dv * pv;
      }
    }
  }
  if constexpr (!DOTS) {
    const int col = c0 + (lane & 15);
    const float bias = P.bias != nullptr && col < P.n ? P.bias[col] : 0.0f;
    int rows[4], cols[4];
    float y[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      rows[v] = r0 + 4 * (lane >> 4) + v;
      cols[v] = col;
      y[v] = s[v] + bias;
    }
    store_tile(P, rows, cols, y);
  }
}

}  // namespace

static unsigned blocks_for(long n, int per) { return (unsigned)((n + per - 1) / per); }

hipError_t launch_quantize(const float* x, int rows, int k, int8_t* q, int ldq, float* scales, uint32_t* nonfinite,
                           hipStream_t s) {
  const long waves = (long)rows * ((k + 255) / 256);
  if (waves == 0) return hipSuccess;
  k_quantize<<<blocks_for(waves, 4), 256, 0, s>>>(x, rows, k, q, ldq, scales, nonfinite);
  return hipGetLastError();
}

hipError_t launch_repack(const uint8_t* values, const float* scales, int n, int k, Weights* w, hipStream_t s) {
  const long chunks = (long)(w->np / 32) * w->g * 2 * 64;
  k_repack_values<<<blocks_for(chunks, 256), 256, 0, s>>>(values, n, k, w->g, w->values, chunks);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_repack_scales<<<blocks_for((long)(w->g + 1) * w->np, 256), 256, 0, s>>>(scales, n, w->g, w->np, w->scales);
  return hipGetLastError();
}

hipError_t launch_export(const Weights* w, uint8_t* values, float* scales, hipStream_t s) {
  k_export_values<<<blocks_for((long)w->n * w->k, 256), 256, 0, s>>>(w->values, w->n, w->k, w->g, values);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_export_scales<<<blocks_for((long)w->n * w->g, 256), 256, 0, s>>>(w->scales, w->n, w->g, w->np, scales);
  return hipGetLastError();
}

hipError_t launch_pad_rows(const int8_t* q, int rows, int k, int8_t* dst, int ldq, hipStream_t s) {
  k_pad_rows<<<blocks_for((long)rows * ldq, 256), 256, 0, s>>>(q, rows, k, dst, ldq);
  return hipGetLastError();
}

#ifndef DQ8_SKINNY16_DEPTH
#define DQ8_SKINNY16_DEPTH 4
#endif
int skinny_cols() { return 16; }
int skinny_row_waves(int m) { return (m + 15) / 16; }
int wide_block_rows() { return 32 * DQ8_WIDE_RT * DQ8_WIDE_WM; }
int wide_block_cols() { return 32 * DQ8_WIDE_CT * DQ8_WIDE_WN; }

hipError_t launch_linear(const Batch& b, int kind, bool dots, hipStream_t s) {
  if (b.total_waves == 0) return hipSuccess;
  if (kind == 0) {
    // total_waves counts blocks for the wide kernel
    constexpr int threads = 64 * DQ8_WIDE_WM * DQ8_WIDE_WN;
    if (dots)
      k_linear_wide<DQ8_WIDE_WM, DQ8_WIDE_WN, DQ8_WIDE_RT, DQ8_WIDE_CT, DQ8_WIDE_STAGES, DQ8_WIDE_CVT_VALU, true>
          <<<b.total_waves, threads, 0, s>>>(b);
    else
      k_linear_wide<DQ8_WIDE_WM, DQ8_WIDE_WN, DQ8_WIDE_RT, DQ8_WIDE_CT, DQ8_WIDE_STAGES, DQ8_WIDE_CVT_VALU, false>
          <<<b.total_waves, threads, 0, s>>>(b);
    return hipGetLastError();
  }
  const unsigned blocks = blocks_for(b.total_waves, 4);
  if (dots) k_linear_skinny16<DQ8_SKINNY16_DEPTH, true><<<blocks, 256, 0, s>>>(b);
  else k_linear_skinny16<DQ8_SKINNY16_DEPTH, false><<<blocks, 256, 0, s>>>(b);
  return hipGetLastError();
}

}  // namespace dq8

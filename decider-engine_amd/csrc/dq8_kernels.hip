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

#include <type_traits>

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
// One 32x32 block with K=2: lanes 0-31 carry k=0 (row / column l), lanes 32-63
// k=1.  With the k=1 operands zero it is the K=1 outer product of one block.
__device__ __forceinline__ v16f mfma_k2(float a, float b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
// 16 outer products of 4 x 4 (v_mfma_f32_4x4x1_16b_f32): block b takes A and
// B from lanes 4b..4b+3, output element v of lane 4b + j is A[v] * B[j]; with
// C = 0 every element is one product rounded once.
__device__ __forceinline__ v4f mfma_k1_4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v32f concat(v16i lo, v16i hi) {
  v16f a = __builtin_bit_cast(v16f, lo), b = __builtin_bit_cast(v16f, hi);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20,
                                 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
}
__device__ __forceinline__ v4i load16(const void* p) { return *reinterpret_cast<const v4i*>(p); }

// 2^(j/32), j = 0..31, correctly rounded to double.
__constant__ double kExp2Frac[32] = {
    0x1.0000000000000p+0, 0x1.059b0d3158574p+0, 0x1.0b5586cf9890fp+0, 0x1.11301d0125b51p+0,
    0x1.172b83c7d517bp+0, 0x1.1d4873168b9aap+0, 0x1.2387a6e756238p+0, 0x1.29e9df51fdee1p+0,
    0x1.306fe0a31b715p+0, 0x1.371a7373aa9cbp+0, 0x1.3dea64c123422p+0, 0x1.44e086061892dp+0,
    0x1.4bfdad5362a27p+0, 0x1.5342b569d4f82p+0, 0x1.5ab07dd485429p+0, 0x1.6247eb03a5585p+0,
    0x1.6a09e667f3bcdp+0, 0x1.71f75e8ec5f74p+0, 0x1.7a11473eb0187p+0, 0x1.82589994cce13p+0,
    0x1.8ace5422aa0dbp+0, 0x1.93737b0cdc5e5p+0, 0x1.9c49182a3f090p+0, 0x1.a5503b23e255dp+0,
    0x1.ae89f995ad3adp+0, 0x1.b7f76f2fb5e47p+0, 0x1.c199bdd85529cp+0, 0x1.cb720dcef9069p+0,
    0x1.d5818dcfba487p+0, 0x1.dfc97337b9b5fp+0, 0x1.ea4afa2a490dap+0, 0x1.f50765b6e4540p+0};

// expf as the reference's f32::exp computes it: Rust lowers it to the libm
// expf of the host, glibc 2.35 on x86-64, whose algorithm (sysdeps/ieee754/
// flt-32/e_expf.c, from ARM's optimized-routines) is restated here in the
// form glibc's FMA build runs (__expf_fma, selected on every x86-64 with
// FMA3):
//   k = round(x * 32/ln2), r = x * 32/ln2 - k (both from one fused
//   multiply-add of x, so r is exact), exp(x) = 2^(k/32) * p(r) with
//   p(r) = (c0 r + c1) r^2 + (c2 r + 1) in double, rounded once to float.
// The rounding to the nearest integer adds and subtracts 1.5 * 2^52; the low
// bits of that sum are k, giving the table index (k mod 32) and the exponent
// (k div 32).  Inputs at or above 89 overflow to +inf and inputs at or below
// -104 round to +0, as in glibc.
__device__ __forceinline__ float expf_libm(float x) {
  if (x != x) return x + x;
  if (x >= 89.0f) return __builtin_inff();
  if (x <= -104.0f) return 0.0f;
  constexpr double kInvLn2x32 = 0x1.71547652b82fep+0 * 32, kShift = 0x1.8p+52;
  constexpr double c0 = 0x1.c6af84b912394p-20, c1 = 0x1.ebfce50fac4f3p-13, c2 = 0x1.62e42ff0c52d6p-6;
  const double xd = x;
  double kd = __builtin_fma(kInvLn2x32, xd, kShift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2x32, xd, -kd);
  const uint32_t j = (uint32_t)ki & 31u;
  const double s = __builtin_bit_cast(double, __builtin_bit_cast(uint64_t, kExp2Frac[j]) + ((ki - j) << 47));
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  return (float)(y * s);
}

// silu (decider-engine src/qwen.rs:194-199): x * (1 / (1 + exp(-x))), each
// operation one fp32 rounding.
__device__ __forceinline__ float silu(float x) {
  const float e = expf_libm(-x);
  return x * (1.0f / (1.0f + e));
}

// The same silu for a whole wave at a time (every lane active; see ExpTab):
//  * expf_libm with the table entry fetched from the wave's registers by
//    ds_bpermute instead of a per-lane constant-memory load, and the three
//    special ranges applied as selects after the arithmetic (their
//    intermediate values are discarded);
//  * 1 / y by v_rcp_f32 and one fused correction r0 + r0 * (1 - y * r0),
//    which equals the IEEE quotient for every float y in [1, 2^126] (checked
//    on gfx950 against the division for all 2^30 of them); above 2^126 the
//    reciprocal is subnormal and y = 1 + e takes the division.
struct ExpTab {
  int lo, hi;  // lane l holds kExp2Frac[l % 32]
  // kShift and c1 of expf_wave: each shares an FMA with another double
  // constant, so one of the two must sit in VGPRs; held here once rather than
  // rebuilt by two moves per call
  double shift, c1;
};
__device__ __forceinline__ ExpTab exp_table(int lane) {
  const uint64_t t = __builtin_bit_cast(uint64_t, kExp2Frac[lane & 31]);
  double shift = 0x1.8p+52, c1 = 0x1.ebfce50fac4f3p-13;
  asm volatile("" : "+v"(shift), "+v"(c1));
  return {(int)(uint32_t)t, (int)(uint32_t)(t >> 32), shift, c1};
}
__device__ __forceinline__ float expf_wave(float x, const ExpTab& T) {
  constexpr double kInvLn2x32 = 0x1.71547652b82fep+0 * 32, kShift = 0x1.8p+52;
  constexpr double c0 = 0x1.c6af84b912394p-20, c2 = 0x1.62e42ff0c52d6p-6;
  const double xd = x;
  double kd = __builtin_fma(kInvLn2x32, xd, T.shift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2x32, xd, -kd);
  const int j = (int)((uint32_t)ki & 31u);
  const uint32_t tlo = (uint32_t)__builtin_amdgcn_ds_bpermute(j << 2, T.lo);
  const uint32_t thi = (uint32_t)__builtin_amdgcn_ds_bpermute(j << 2, T.hi);
  const uint64_t tb = ((uint64_t)thi << 32) | tlo;
  const double sc = __builtin_bit_cast(double, tb + ((ki - (uint64_t)j) << 47));
  const double z = __builtin_fma(c0, r, T.c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  float v = (float)(y * sc);
  // The special ranges (and NaN) are rare: their selects run only when some
  // lane of the wave needs them (a wave-uniform branch).
  if (__ballot(!(x > -104.0f && x < 89.0f)) != 0) {
    asm volatile("");  // keeps the compiler from evaluating the selects unconditionally
    v = x >= 89.0f ? __builtin_inff() : v;
    v = x <= -104.0f ? 0.0f : v;
    v = x != x ? x + x : v;
  }
  return v;
}
__device__ __forceinline__ float silu_wave(float x, const ExpTab& T) {
  const float y = 1.0f + expf_wave(-x, T);
  const float r0 = __builtin_amdgcn_rcpf(y);
  float rq = __builtin_fmaf(__builtin_fmaf(-y, r0, 1.0f), r0, r0);
  // subnormal reciprocal, inf or NaN: the division, only when some lane of
  // the wave has such a y (otherwise the compiler evaluates it for every lane)
  if (__ballot(!(y <= 0x1p126f)) != 0) rq = !(y <= 0x1p126f) ? 1.0f / y : rq;
  return x * rq;
}

#ifndef DQ8_NT_OUT
#define DQ8_NT_OUT 1
#endif
// One fp32 output store.  Outputs are written once and never re-read by the
// kernel that writes them, so the stores are marked non-temporal (build with
// -DDQ8_NT_OUT=0 for plain stores); the bits stored are the same either way.
__device__ __forceinline__ void st_out(float* p, float v) {
#if DQ8_NT_OUT
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
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
      if (row[e] < P.m && col[e] < P.n) st_out(P.out + (size_t)col[e] * P.m + row[e], y[e]);
    return;
  }
  if (P.epilogue == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (row[e] < P.m && col[e] < P.n) st_out(P.out + (size_t)row[e] * P.n + col[e], y[e]);
    return;
  }
  float old[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    old[e] = row[e] < P.m && col[e] < P.n ? P.out[(size_t)row[e] * P.n + col[e]] : 0.0f;
  if (P.epilogue == 1) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (row[e] < P.m && col[e] < P.n) st_out(P.out + (size_t)row[e] * P.n + col[e], old[e] + y[e]);
    return;
  }
  // SwiGlu: each silu with all lanes active, then its store; a few elements
  // at a time, so the f64 temporaries of only those are live
  const ExpTab T = exp_table((int)(threadIdx.x & 63));
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float sv = silu_wave(old[e], T);
    if (row[e] < P.m && col[e] < P.n) st_out(P.out + (size_t)row[e] * P.n + col[e], sv * y[e]);
    if ((e & 3) == 3) __builtin_amdgcn_sched_barrier(0);
  }
}

// store_tile for E values of a tile inside m x n in the rows layout: value e
// at row ur[e], column uc[e] (wave-uniform) plus the lane's fixed byte offset
// loff, so no bounds checks and no per-value address arithmetic on the VALU.
template <int E>
__device__ __forceinline__ void store_tile_full(const Proj& P, const int (&ur)[E], const int (&uc)[E], uint32_t loff,
                                                const float (&y)[E]) {
  auto at = [&](int e) {
    return reinterpret_cast<float*>(reinterpret_cast<char*>(P.out + (size_t)ur[e] * P.n + uc[e]) + loff);
  };
  if (P.epilogue == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) st_out(at(e), y[e]);
    return;
  }
  float old[E];
#pragma unroll
  for (int e = 0; e < E; ++e) old[e] = *at(e);
  if (P.epilogue == 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) st_out(at(e), old[e] + y[e]);
    return;
  }
  const ExpTab T = exp_table((int)(threadIdx.x & 63));
#pragma unroll
  for (int e = 0; e < E; ++e) {
    st_out(at(e), silu_wave(old[e], T) * y[e]);
    if ((e & 3) == 3) __builtin_amdgcn_sched_barrier(0);
  }
}

// The projection of a launch's block: the last one whose first block is at
// most `wave`.  UNROLL: over the batch's fixed capacity and the contiguous
// copy of the first blocks, so the kernel argument loads are one or two
// instructions with one latency rather than one round trip per item: the
// skinny kernel's grouped launches of 9 projections start 2 us sooner (the
// wide kernel's launches hold 1 to 3 and measured slower with the per-item
// form of this).
template <bool UNROLL = false>
__device__ __forceinline__ int find_proj(const Batch& b, int wave) {
  int pi = 0;
  if constexpr (UNROLL) {
#pragma unroll
    for (int i = 1; i < kMaxBatch; ++i)
      if (i < b.count && wave >= b.wave_begin[i]) pi = i;
  } else {
    for (int i = 1; i < b.count; ++i)
      if (wave >= b.p[i].wave_begin) pi = i;
  }
  return pi;
}

// LoRA term of Adapter::combine (tensor.rs:109-117) for one MFMA tile set:
// out = base + scale * (dot_scores(mid[row], b[col]) + 0.0), dot_scores in its
// x86-64 order (tensor.rs:6-25): lane i of 8 sums the products of elements i,
// i+8, ...; the lanes are added in order, then the tail elements one by one.
// prod(i) returns the tile's products mid[row][i] * b[col][i] (each one rounded
// product, from a K=1 MFMA with C = 0).  The reference starts its lanes at 0.0
// and their sum at -0.0; starting from the first product instead only changes
// the sign of an all-zero partial sum, and the final + 0.0 makes every zero
// delta +0.0 in both, so the result is identical.
template <typename V, typename Prod>
__device__ __forceinline__ V lora_term(const V& base, const V& zero, int rank, float scale, Prod prod) {
  const int chunks = rank >> 3;
  V sum = zero;  // no full chunk: eight +0.0 lanes sum to +0.0
  if (chunks > 0) {
    for (int i = 0; i < 8; ++i) {
      V ln = prod(i);
      for (int c = 1; c < chunks; ++c) ln = ln + prod(8 * c + i);
      sum = i == 0 ? ln : sum + ln;
    }
  }
  for (int t = 8 * chunks; t < rank; ++t) sum = sum + prod(t);
  return base + scale * (sum + zero);
}

// lora_term for rank <= 16 with every index a compile-time constant after
// unrolling, so the operands can sit in registers, loaded up front.
template <typename V, typename Prod>
__device__ __forceinline__ V lora_term16(const V& base, const V& zero, int rank, float scale, Prod prod) {
  const int chunks = rank >> 3;
  V sum = zero;
  if (chunks > 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      V ln = prod(i);
      if (chunks > 1) ln = ln + prod(8 + i);
      sum = i == 0 ? ln : sum + ln;
      __builtin_amdgcn_sched_barrier(0);  // keeps the products of one lane live at a time
    }
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    if (t >= 8 * chunks && t < rank) sum = sum + prod(t);
    __builtin_amdgcn_sched_barrier(0);
  }
  return base + scale * (sum + zero);
}

// LDS staging of lora_block32: 64 rows of kLoraRow floats per wave.
constexpr int kLoraRow = 17;
constexpr int kLoraStage = 64 * kLoraRow * 4;

// Adapter term of one 32 x 32 block of a wave (rows mw .. mw+31, columns cb ..
// cb+31; element v of lane l at row mw + 8(v/4) + 4(l/32) + v%4, column
// cb + l%32): base + scale * (dot_scores(mid[row], b[col]) + 0.0), the same
// arithmetic as the adapter epilogue of k_linear_wide.  For rank 16 the wave
// first copies its 32 mid rows and 32 b rows into its own kLoraStage bytes of
// LDS (lw; rows padded to 17 floats, so the 32 b rows one operand read touches
// sit in distinct banks and every read is a base register plus an immediate
// offset), then forms the products with v_mfma_f32_4x4x1_16b_f32 in 4 slices
// of 4 rows.  Only ranks 0 and 16 (with
// 16-byte aligned mid and b) come here: the host sends other adapters of a
// gate/up pair to separate launches, whose epilogue takes any rank.
__device__ __forceinline__ v16f lora_block32(v16f base, const float* lmid, const float* lb, int rank, float scale,
                                             int m, int n, int mw, int cb, int lane, float* lw) {
  v16f zero16;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero16[i] = 0.0f;
  if (rank == 0) return base + scale * (zero16 + zero16);  // no products: a +0.0 dot
  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  float* lmw = lw;                  // rows 0-31: mid
  float* lbw = lw + 32 * kLoraRow;  // rows 32-63: b
  // Both operand runs are contiguous (32 * 16 floats each); rows past m or n
  // read the last row instead.
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int e = 64 * t + lane;  // float4 index: row e/4, inputs 4(e%4)..+3
    const v4f vm = *reinterpret_cast<const v4f*>(lmid + (size_t)min(mw + (e >> 2), m - 1) * 16 + 4 * (e & 3));
    const v4f vb = *reinterpret_cast<const v4f*>(lb + (size_t)min(cb + (e >> 2), n - 1) * 16 + 4 * (e & 3));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lmw[(e >> 2) * kLoraRow + 4 * (e & 3) + q] = vm[q];
      lbw[(e >> 2) * kLoraRow + 4 * (e & 3) + q] = vb[q];
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's copies are visible to it
  const int c = lane & 31;
  const float* rb = lbw + kLoraRow * c;
  const float* rm0 = lmw + kLoraRow * (4 * (lane >> 5) + (lane & 3));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float* rm = rm0 + 8 * kLoraRow * u;  // row 8u + 4(lane/32) + lane%4
    auto prod = [&](int i) { return mfma_k1_4(rm[i], rb[i], zero4); };
    v4f su;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4f ln = prod(i) + prod(8 + i);
      su = i == 0 ? ln : su + ln;
      // keeps the scheduler from issuing every product of the block at once:
      // the pair kernel holds both 32 x 32 accumulators here
      if ((i & 1) == 1) __builtin_amdgcn_sched_barrier(0);
    }
    // a slice's 4 elements are final: combine them now (elementwise, so the
    // same arithmetic as combining the whole block at the end)
#pragma unroll
    for (int v = 0; v < 4; ++v) base[4 * u + v] = base[4 * u + v] + scale * (su[v] + 0.0f);
  }
  return base;
}

// ---------------------------------------------------------------------------
// Stored weight elements (Data::read, weights.rs:147-195): little-endian F32,
// BF16 (the upper half of an F32) or F16.  Both 16-bit decodings are exact:
// bf16 -> f32 is f32::from_bits(v << 16) (weights.rs:38-41) and f16 -> f32 is
// the IEEE conversion that `half` (weights.rs:367-382) spells out.
template <int DT>
__device__ __forceinline__ float decode(const void* base, size_t i) {
  if constexpr (DT == kDtypeF32) {
    return static_cast<const float*>(base)[i];
  } else {
    const uint16_t h = static_cast<const uint16_t*>(base)[i];
    if constexpr (DT == kDtypeBF16) return __builtin_bit_cast(float, (uint32_t)h << 16);
    else return (float)__builtin_bit_cast(_Float16, h);
  }
}
// The quantizer's fp32 input is read once, and its bytes and scales go to
// memory anyway (the next kernel reads them from other XCDs' L2s), so its
// loads and stores are non-temporal: the 2048-row stack's 72 calls of 2048 x
// 2048 took 0.419 against 0.460 ms, graph-replayed alone.
#ifndef DQ8_QUANT_NT
#define DQ8_QUANT_NT 1
#endif
#ifndef DQ8_QUANT_NTS
#define DQ8_QUANT_NTS 1
#endif
template <int DT>
__device__ __forceinline__ void decode4(const void* base, size_t i, float (&v)[4]) {
  if constexpr (DT == kDtypeF32) {
#if DQ8_QUANT_NT
    const v4f t4 = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(static_cast<const float*>(base) + i));
    v[0] = t4[0]; v[1] = t4[1]; v[2] = t4[2]; v[3] = t4[3];
#else
    const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
#endif
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
    const uint16_t h[4] = {(uint16_t)t.x, (uint16_t)(t.x >> 16), (uint16_t)t.y, (uint16_t)(t.y >> 16)};
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = decode<DT>(h, j);
  }
}

// Lane permutations by DPP (no LDS round trip): quad_perm [1,0,3,2] and
// [2,3,0,1], and rotations by 4 and 8 lanes within each row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
// Max over each aligned group of 4 lanes, and of 16 lanes, of non-negative,
// non-NaN floats (absmax partials that start from 0.0f through fmaxf): their
// bit patterns order as the values do.
__device__ __forceinline__ float max_quad(float m) {
  uint32_t b = __builtin_bit_cast(uint32_t, m);
  b = max(b, dpp<0xB1>(b));
  b = max(b, dpp<0x4E>(b));
  return __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_row16(float m) {
  uint32_t b = __builtin_bit_cast(uint32_t, max_quad(m));
  b = max(b, dpp<0x124>(b));
  b = max(b, dpp<0x128>(b));
  return __builtin_bit_cast(float, b);
}

// One group's scale from its absmax m (weights.rs:117-136): absmax / 127, at
// least FLT_MIN, 1 for an all-zero group.
__device__ __forceinline__ float quant_scale(float m) {
  return (m == 0.0f) ? 1.0f : fmaxf(m / 127.0f, FLT_MIN);
}
// The same scale with fewer instructions: for m in [2^-100, FLT_MAX] the IEEE
// quotient m / 127 is q0 + r * c rounded once, with c = 1/127 rounded, q0 = m *
// c rounded and r = m - 127 * q0 exact (one FMA); the quotient is then above
// FLT_MIN.  That equals m / 127 for every float in the range (checked
// exhaustively on the CPU by tests/test_scale_division.py).  Other m divide.
__device__ __forceinline__ float quant_scale_fma(float m) {
  constexpr float c = 1.0f / 127.0f;
  if (m >= 0x1p-100f && m <= FLT_MAX) {
    const float q0 = m * c;
    return __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, m), c, q0);
  }
  return quant_scale(m);
}
// N elements of one group: round(v / scale) half away from zero (f32::round of
// the IEEE quotient), as int8 in [-127, 127], packed 4 bytes to a word.
// The quotient is taken through rs = rcp(scale) (1 ulp): a = v * rs differs from
// the IEEE quotient Q by less than 2^-15 (|Q| <= 127, relative error < 2^-22).
// u = a + 128 is within 2^-17 of the exact sum, so when u lies more than 2^-14
// from every half-integer, rint(u) = round(Q) + 128, an integer in [1, 255]
// (|a| < 127.0001, no clamp needed), converted and packed by v_cvt_pk_u8_f32;
// the XOR with 0x80 turns it into the two's complement byte.  A wave with an
// element closer than that (about 1 in 8000 elements) divides all its
// elements exactly.
// FMA: u = v * rs + 128 rounded once instead of twice; u is then within 2^-16
// + 2^-17 of Q + 128, inside the same margin.
template <int N, bool FMA = false>
__device__ __forceinline__ void quant_pack(const float (&v)[N], float scale, uint32_t (&w)[N / 4]) {
  const float rs = __builtin_amdgcn_rcpf(scale);
  float r[N];
  float fm = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float u = FMA ? __builtin_fmaf(v[i], rs, 128.0f) : v[i] * rs + 128.0f;
    r[i] = rintf(u);
    fm = fmaxf(fm, fabsf(u - r[i]));
  }
  // Some element within 2^-14 of a rounding boundary: the exact quotients,
  // decided per wave (they equal the shortcut wherever the margin holds), so
  // the divisions run only in such waves instead of in every lane, selected.
  if (__ballot(!(0.5f - fm > 0x1p-14f)) != 0) {
    asm volatile("");  // keeps the divisions inside the branch
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = fminf(fmaxf(roundf(v[i] / scale), -127.0f), 127.0f) + 128.0f;
  }
#pragma unroll
  for (int j = 0; j < N / 4; ++j) {
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) x = __builtin_amdgcn_cvt_pk_u8_f32(r[4 * j + i], i, x);
    w[j] = x ^ 0x80808080u;
  }
}

// Quantization: QuantizedInputs::new (tensor.rs:321-339) and the 8-bit
// Data::quantize (weights.rs:117-136).  A wave covers PER consecutive
// 256-element chunks of one row (4 elements per lane and chunk, 4 groups per
// chunk); every chunk's load is issued before the first is used, so a wave
// keeps PER KB (fp32) in flight.  A group's absmax is a max-reduction over its
// 16 lanes; quant_pack rounds the elements (the IEEE quotient by the scale,
// half away from zero, as f32::round).  x holds DT elements; a non-finite one ORs 1 into
// *nonfinite (Data::read rejects it for weights, QuantizedInputs::new returns
// None for inputs).  The host guarantees rows * ceil(chunks / PER) < 2^31 and
// passes wdiv, the divider by the waves per row (wave / wpr without a division).
#ifndef DQ8_QUANT_WPB
#define DQ8_QUANT_WPB 4
#endif
template <int DT, int PER>
__global__ __launch_bounds__(64 * DQ8_QUANT_WPB) void k_quantize(const void* __restrict__ x, int rows, int k, int8_t* __restrict__ q,
                                                  int ldq, float* __restrict__ scales, int lds, uint32_t* nonfinite,
                                                  Divider wdiv) {
  const int lane = threadIdx.x & 63;
  const int chunks = (k + 255) >> 8;
  const int wpr = (chunks + PER - 1) / PER;  // waves per row
  const int wave = blockIdx.x * DQ8_QUANT_WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = wdiv.div((uint32_t)wave);
  if (row >= rows) return;  // wave-uniform
  const int c0 = (wave - row * wpr) * PER;
  const bool vec = (k & 3) == 0 && ((uintptr_t)x & (DT == kDtypeF32 ? 15 : 7)) == 0;
  const size_t r0 = (size_t)row * k;
  int8_t* qr = q + (size_t)row * ldq;
  const bool qvec = (ldq & 3) == 0 && ((uintptr_t)q & 3) == 0;
  const int groups = (k + kGroup - 1) / kGroup;
  // Scales and bytes of the wave's chunks; true if an element is not finite.
  // whole: every chunk lies in the row and the bytes can be stored as words.
  auto finish = [&](const float (&v)[PER][4], auto whole) {
    bool bad = false;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int chunk = c0 + p;
      if (!whole && chunk >= chunks) break;  // wave-uniform
      const int k0 = chunk * 256 + lane * 4;
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bad |= !isfinite(v[p][i]);
        m = fmaxf(m, fabsf(v[p][i]));
      }
      m = max_row16(m);  // over the 16 lanes of this group
      const float scale = quant_scale(m);
      uint32_t pk[1];
      quant_pack<4>(v[p], scale, pk);
      const uint32_t packed = pk[0];
      if (whole || (qvec && k0 + 3 < ldq)) {
        // Padding bytes [k, ldq) are written as zero (v = 0 there).
#if DQ8_QUANT_NTS
        __builtin_nontemporal_store(packed, reinterpret_cast<uint32_t*>(qr + k0));
#else
        *reinterpret_cast<uint32_t*>(qr + k0) = packed;
#endif
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + i < ldq) qr[k0 + i] = (int8_t)(packed >> (8 * i));
      }
      const int group = chunk * 4 + (lane >> 4);
#if DQ8_QUANT_NTS
      if ((lane & 15) == 0 && (whole || group < groups))
        __builtin_nontemporal_store(scale, scales + (size_t)row * lds + group);
#else
      if ((lane & 15) == 0 && (whole || group < groups)) scales[(size_t)row * lds + group] = scale;
#endif
    }
    return bad;
  };
  float v[PER][4];
  bool bad;
  if (vec && qvec && (c0 + PER) * 256 <= k) {
    // Every chunk of the wave is whole (wave-uniform): plain loads with no
    // lane condition, all issued first (the empty asm keeps the compiler from
    // sinking them), and the chunks are finished on this path, so each one
    // waits for its own load only (loads under a lane-divergent branch make
    // the compiler wait for all of them where the paths join).
#pragma unroll
    for (int p = 0; p < PER; ++p) decode4<DT>(x, r0 + (c0 + p) * 256 + lane * 4, v[p]);
    asm volatile("" ::: "memory");
    bad = finish(v, std::true_type{});
  } else {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int k0 = (c0 + p) * 256 + lane * 4;  // chunks past the row's end: k0 >= k, all zeros, not stored
      if (vec && k0 + 3 < k) {
        decode4<DT>(x, r0 + k0, v[p]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[p][i] = (k0 + i < k) ? decode<DT>(x, r0 + k0 + i) : 0.0f;
      }
    }
    bad = finish(v, std::false_type{});
  }
  if (nonfinite) {  // one atomic per wave that saw a non-finite element
    const unsigned long long b = __ballot(bad);
    if (b != 0 && lane == __builtin_ffsll((long long)b) - 1) atomicOr(nonfinite, 1u);
  }
}

// The fp32 quantizer for rows of whole chunks (k % 256 == 0, 16-byte aligned x,
// 4-byte aligned q rows): the same bytes and scales as k_quantize, from a grid
// of at most kQuantLoopBlocks blocks whose waves walk the chunks (global chunk
// c = row * (k / 256) + chunk of the row; wave w takes w, w + W, w + 2W, ...
// for W waves) with D loads in flight: a chunk's slot is reloaded before the
// chunk is finished.  Fewer, longer-lived waves keep more bytes in flight per wave than
// one chunk per wave (2048 x 2048 fp32: a copy of the same bytes takes 4.8
// against 5.3 us per call at one 1 KB load per wave, graph-replayed).
#ifndef DQ8_QUANT_LOOP_BLOCKS
#define DQ8_QUANT_LOOP_BLOCKS 1536
#endif
constexpr int kQuantLoopBlocks = DQ8_QUANT_LOOP_BLOCKS;
#ifndef DQ8_QUANT_LOOP_NT_SCALES
#define DQ8_QUANT_LOOP_NT_SCALES 1
#endif
#ifndef DQ8_QUANT_LOOP_BITS
#define DQ8_QUANT_LOOP_BITS 1
#endif
#ifndef DQ8_QUANT_LOOP_FMA
#define DQ8_QUANT_LOOP_FMA 1
#endif
#ifndef DQ8_QUANT_LOOP
#define DQ8_QUANT_LOOP 2  // chunks in flight per wave (0: one chunk per wave, k_quantize)
#endif
#ifndef DQ8_QUANT_LOOP_WPB
#define DQ8_QUANT_LOOP_WPB 4
#endif
template <int D>
__global__ __launch_bounds__(64 * DQ8_QUANT_LOOP_WPB) void k_quantize_loop(const float* __restrict__ x, int k, int total,
                                                       int8_t* __restrict__ q, int ldq, float* __restrict__ scales,
                                                       int lds, uint32_t* nonfinite, Divider cdiv) {
  const int lane = threadIdx.x & 63;
  const int W = (int)gridDim.x * DQ8_QUANT_LOOP_WPB;
  const int w = (int)blockIdx.x * DQ8_QUANT_LOOP_WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cpr = k >> 8;
  auto load = [&](int c, float (&v)[4]) {
    const int row = cdiv.div((uint32_t)c);
    decode4<kDtypeF32>(x, (size_t)row * k + (size_t)(c - row * cpr) * 256 + lane * 4, v);
  };
  float v[D][4];
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (w + d * W < total) load(w + d * W, v[d]);  // wave-uniform
  bool bad = false;
  for (int c0 = w; c0 < total; c0 += D * W) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int c = c0 + d * W;
      if (c >= total) break;  // wave-uniform
      const int row = cdiv.div((uint32_t)c), chunk = c - row * cpr;
      float e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = v[d][i];
      // the slot's next load goes out before this chunk is finished (the empty
      // asm keeps it there)
      const int cn = c + D * W;
      if (cn < total) load(cn, v[d]);  // wave-uniform
      asm volatile("" ::: "memory");
#if DQ8_QUANT_LOOP_BITS
      // absmax and the finite check from the magnitudes' bit patterns: they
      // order as the values do, and a NaN or an infinity has the largest
      // exponent.  A NaN (only with the non-finite flag set, when the bytes are
      // not used) then makes the scale NaN, where fmaxf would skip it.
      uint32_t mb = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) mb = max(mb, __builtin_bit_cast(uint32_t, e[i]) & 0x7fffffffu);
      bad |= mb >= 0x7f800000u;
      const float m = max_row16(__builtin_bit_cast(float, mb));
#else
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bad |= !isfinite(e[i]);
        m = fmaxf(m, fabsf(e[i]));
      }
      m = max_row16(m);  // over the 16 lanes of this group
#endif
#if DQ8_QUANT_LOOP_FMA
      const float scale = quant_scale_fma(m);
      uint32_t pk[1];
      quant_pack<4, true>(e, scale, pk);
#else
      const float scale = quant_scale(m);
      uint32_t pk[1];
      quant_pack<4>(e, scale, pk);
#endif
#if DQ8_QUANT_NTS
      __builtin_nontemporal_store(pk[0], reinterpret_cast<uint32_t*>(q + (size_t)row * ldq + chunk * 256 + lane * 4));
#if DQ8_QUANT_LOOP_NT_SCALES
      if ((lane & 15) == 0) __builtin_nontemporal_store(scale, scales + (size_t)row * lds + chunk * 4 + (lane >> 4));
#else
      if ((lane & 15) == 0) scales[(size_t)row * lds + chunk * 4 + (lane >> 4)] = scale;
#endif
#else
      *reinterpret_cast<uint32_t*>(q + (size_t)row * ldq + chunk * 256 + lane * 4) = pk[0];
      if ((lane & 15) == 0) scales[(size_t)row * lds + chunk * 4 + (lane >> 4)] = scale;
#endif
    }
  }
  if (nonfinite) {  // one atomic per wave that saw a non-finite element
    const unsigned long long b = __ballot(bad);
    if (b != 0 && lane == __builtin_ffsll((long long)b) - 1) atomicOr(nonfinite, 1u);
  }
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
// xs [rows][g] -> dst [rows][ld] (ld >= g), zero past g.
__global__ void k_pad_scales(const float* __restrict__ xs, int rows, int g, float* __restrict__ dst, int ld) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * ld) return;
  const int row = (int)(i / ld), c = (int)(i - (long)row * ld);
  dst[i] = c < g ? xs[(size_t)row * g + c] : 0.0f;
}

__global__ void k_pad_rows(const int8_t* __restrict__ q, int rows, int k, int8_t* __restrict__ dst, int ldq) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * ldq) return;
  const int row = (int)(i / ldq), kk = (int)(i % ldq);
  dst[i] = kk < k ? q[(size_t)row * k + kk] : (int8_t)0;
}

// ---------------------------------------------------------------------------
// Wide projection kernel (M > 32): helpers.

// Tile (row tile mt, column tile nt) of block i of a projection.  Blocks are
// dealt to the 8 XCDs round robin, so blocks i, i+8, ... share one XCD and its
// L2.  With P.xcd_gm = gm the tile grid is cut into gm x (8/gm) regions and
// XCD i%8 walks region i%8: it touches 1/gm of the activation rows and
// 1/(8/gm) of the weight columns.  Within its region an XCD takes bands of
// sr = P.xcd_sr row tiles, and each band in chunks of sc = P.xcd_sc column
// tiles, row tiles fastest, so the blocks that run at the same time share sr
// row tiles of activations and sc column tiles of weights in L2.  The map is a
// bijection on [0, row_tiles * col_tiles) (the host picks gm dividing both
// counts and sr dividing the region's row tiles).
// The divisions are multiply-shifts by host-computed Dividers (scalar ALU
// only).
__device__ __forceinline__ void tile_of(const Proj& P, int i, int& mt, int& nt) {
  if (P.xcd_gm == 0) {
    mt = P.d_cols.div((uint32_t)i);
    nt = i - mt * P.waves_n;
    return;
  }
  const int rm = P.xcd_rm, rn = P.xcd_rn;  // region size in tiles
  const int x = i & 7, j = i >> 3;
  const int xa = x >> P.xcd_gn_shift, xb = x - (xa << P.xcd_gn_shift);
  const int sr = P.xcd_sr, sc = P.xcd_sc;
  const int band = P.d_band.div((uint32_t)j), t = j - band * (sr * rn);
  const int chunk = P.d_chunk.div((uint32_t)t), u = t - chunk * (sr * sc);
  const int uq = P.d_sr.div((uint32_t)u), ur = u - uq * sr;
  mt = xa * rm + band * sr + ur;
  nt = xb * rn + chunk * sc + uq;
}

// Direct global->LDS loads.  They are issued through inline assembly so the
// compiler does not track them: its LDS-DMA bookkeeping is conservative at
// loop headers and would drain the whole pipeline there.  The kernel orders
// every use itself (wait_vmcnt + s_barrier).  No compiler-generated code in
// these kernels uses M0; the s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}
// The address is split into a wave-uniform 64-bit base (SGPRs, advanced per
// group on the scalar unit) and a fixed 32-bit per-lane offset.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, const void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_offset(lds)), "v"(off), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t off, const void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(lds_offset(lds)), "v"(off), "s"(base)
               : "memory");
}
// Block barrier for LDS data: this wave's LDS writes are complete, then
// s_barrier.  Unlike __syncthreads() it does not wait for outstanding global
// loads, so register prefetch rings keep their loads in flight across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Launch shape of the wide kernel (tunable at build time): WM x WN waves per
// block, each wave (32*RT) rows x (32*CT) columns; STAGES groups in flight in
// LDS where the rings are not split (below); x-scale chunk of XCH groups
// there; A-slab swizzle SWZ (0: for 16-lane LDS
// phases, 1: for 8-lane); WPE > 0 caps registers for that many waves per SIMD.
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
#define DQ8_WIDE_STAGES 2
#endif
#ifndef DQ8_WIDE_XCH
#define DQ8_WIDE_XCH 16
#endif
#ifndef DQ8_WIDE_SWZ
#define DQ8_WIDE_SWZ 1
#endif
#ifndef DQ8_WIDE_WPE
#define DQ8_WIDE_WPE 0
#endif
// > 0: the wide kernel runs as a grid of at most DQ8_WIDE_PERSIST blocks per CU
// (256 CUs) that walk the tiles; 0: one block per tile.
#ifndef DQ8_WIDE_PERSIST
#define DQ8_WIDE_PERSIST 0
#endif
// 256-element chunks per wave of the quantizer.
#ifndef DQ8_QUANT_PER
#define DQ8_QUANT_PER 1
#endif
// Launches of at most DQ8_WIDE_DEEP_BLOCKS blocks (at most three per CU, where
// the deeper ring's LDS costs no occupancy), and launches of at most
// DQ8_WIDE_DEEP_MIXED blocks that mix long and short K, use a ring of
// STAGES + 1 groups.  DQ8_WIDE_SPLIT selects the rings of the other launches:
// 0: STAGES groups for A and B; 1: split rings, A for 2 groups and B for 3
// (37.5 KB with 8-group x chunks, so 4 blocks still fit a CU); 2: split rings
// for every launch.
#ifndef DQ8_WIDE_SPLIT
#define DQ8_WIDE_SPLIT 1
#endif
#ifndef DQ8_WIDE_DEEP_BLOCKS
#define DQ8_WIDE_DEEP_BLOCKS 768
#endif
#ifndef DQ8_WIDE_DEEP_MIXED
#define DQ8_WIDE_DEEP_MIXED 1533
#endif
// Launches of at most DQ8_WIDE_DEEP4_BLOCKS blocks (two per CU) use a ring of
// 4 groups (58 KB of LDS): down (2048 x 6144 -> 2048) 58.7 -> 56.2 us, the
// 2048 x 2048 -> 2048 launches unchanged; a ring of 5 was slower (59.8 us).
#ifndef DQ8_WIDE_DEEP4_BLOCKS
#define DQ8_WIDE_DEEP4_BLOCKS 512
#endif

// ---------------------------------------------------------------------------
// Wide projection kernel (M > 32), LDS-staged.  A block of WM x WN waves owns
// a (32*RT*WM) x (32*CT*WN) output tile; each wave owns (32*RT) x (32*CT) of
// it.  Per group, a wave's 32x32 tiles are processed in pairs that share one
// conversion MFMA and one product MFMA (blocks 0 and 1 of
// v_mfma_f32_32x32x1_2b_f32):
//   RT == 2: pair j = row tiles (0, 1) at column tile j;  A lane l: x of row l,
//            B lane l: w of column 32j + l%32.
//   RT == 1: one pair = column tiles (0, 1) at the single row tile;  A lane l:
//            x of row l%32, B lane l: w of column l.
//
// Operands reach LDS by direct global->LDS loads (global_load_lds_*: lane l's
// bytes land at base + size*l).  The cost of such a load is set by the number
// of distinct cache lines its 64 lanes touch, not by its bytes, so:
//  * A: per group, 16-row x 64-byte slabs (16 lines per 1 KB load).  Lane l of
//    the load fetches row l/4, 16-byte chunk (l%4) ^ f(row) and lands at slot
//    l, so the MFMA operand reads (row R, chunk c) from slot
//    4*(R%16) + (c ^ f(R%16)) of slab R/16: the XOR keeps ds_read_b128 free of
//    bank conflicts (f = (r>>2)&3 for 16-lane phases, (r>>1)&3 for 8-lane).
//  * x scales: once per XCH groups, as row slabs of XCH*4 bytes (one load
//    covers 256/XCH rows), double-buffered; pieces of 4 groups are XOR-swizzled
//    by row like the A chunks.  Pieces past G load an in-bounds dummy (G % 4
//    == 0 and ldxs % 4 == 0 are required; the host pads xs otherwise).
//  * B: 1 KB weight fragments (8 lines each) and w scales (contiguous).
// Every wave issues the same number of loads per group (the last slot is
// padded with a duplicate w-scale load), so the vmcnt waits are compile-time
// constants; an x-scale chunk is issued just before the group loads of its
// first group and is therefore complete when that group is.
//
// Two LDS rings: A slabs of SA groups, B fragments and w scales of SB groups
// (SA == SB, or SA = 2 and SB = 3).  Iteration g: wait for this wave's loads
// of group g, barrier (every wave's loads of group g have landed and every
// wave is done reading group g-1), issue A of group g+SA-1 and then B of group
// g+SB-1 into group g-1's slots, then read group g and compute.  The wait is
// vmcnt <= the loads issued after group g's: with SA == SB the loads of the
// SB-2 newer groups; with SA = 2 < SB the B loads of iteration g-1 (issued
// after A of group g; B of group g is older).  Groups past the end load
// clamped operands and the all-zero w-scale row G; they are never computed on.
// The SwiGLU pair mode needs waves of one 32-row tile and two 32-column tiles
// (gate and up), two waves across: a block then covers 64 whole h columns.
constexpr bool wide_pair_shape(int WN, int RT, int CT) { return RT == 1 && CT == 2 && WN == 2; }
#if DQ8_WIDE_WPE > 0
#define DQ8_WIDE_ATTR __attribute__((amdgpu_waves_per_eu(DQ8_WIDE_WPE, DQ8_WIDE_WPE)))
#else
#define DQ8_WIDE_ATTR
#endif
template <int WM, int WN, int RT, int CT, int SA, int SB, int XCH, int SWZ, bool DOTS, bool LORA, bool PL = false>
__global__ __launch_bounds__(64 * WM * WN) DQ8_WIDE_ATTR void k_linear_wide(Batch b) {
  constexpr int NW = WM * WN, WR = 32 * RT, WC = 32 * CT;
  constexpr int BM = WR * WM, BN = WC * WN;
  constexpr int AS = BM / 16;                  // A slabs per group
  constexpr int BF = BN / 16;                  // B fragments per group
  constexpr int WSD = DOTS ? 0 : BN / 64;      // w-scale loads per group
  constexpr int L16 = (AS + BF) / NW;          // 16-byte loads per wave per group
  constexpr int KA = AS / NW;                  // ... of them A slabs (slots 0 .. KA-1)
  constexpr int LB = L16 - KA + (DOTS ? 0 : 1);  // B loads per wave per group, with the w-scale load
  constexpr int PPR = XCH / 4;                 // 16-byte x-scale pieces per row
  constexpr int RPD = 64 / PPR;                // rows per x-scale load
  constexpr int XD = BM / RPD;                 // x-scale loads per chunk
  constexpr int XPW = (XD + NW - 1) / NW;       // ... per wave (waves 0 .. XD-1 when XD < NW)
  constexpr int NP = RT == 2 ? CT : 1;         // tile pairs per wave
  // Loads of this wave that may still be in flight when group g is computed:
  // with SA == SB the LOADS of each of the SB-2 newer groups; with SA = 2 < SB
  // the B loads of the last iteration, which were issued after A(g).
  constexpr int WAITN = SA == SB ? (SB - 2) * (KA + LB) : LB;
  constexpr int PERIOD = SA == SB ? SA : SA * SB;  // ring slots repeat after PERIOD groups
  static_assert((AS + BF) % NW == 0 && AS % NW == 0, "16-byte loads must split evenly over the waves");
  static_assert(WSD <= NW && (XD % NW == 0 || NW % XD == 0), "scale loads per wave");
  static_assert(XCH == 8 || XCH == 16 || XCH == 32, "x-scale chunk");
  static_assert((RT == 2 && (CT == 1 || CT == 2)) || (RT == 1 && CT == 2), "supported wave tiles");
  static_assert(((SA == SB && SB >= 2 && SB <= 4) || (SA == 2 && SB == 3)) && WAITN + XPW <= 63, "pipeline depth");
  // The LDS rings: A slabs of SA groups, B fragments and w scales of SB groups.
  struct AStage {
    uint8_t frag[AS][kFragBytes];
  };
  struct BStage {
    uint8_t frag[BF][kFragBytes];
    float ws[BN];
  };
  struct Ring {
    AStage a[SA];
    BStage b[SB];
  };
  struct XChunk {
    uint8_t d[XD][kFragBytes];
  };
  __shared__ __attribute__((aligned(16))) Ring ring;
  __shared__ __attribute__((aligned(16))) XChunk xc[DOTS ? 1 : 2];
  // Non-finite inputs (*b.unless != 0): the FP32 kernel runs instead.  The
  // flag is read once a tile's first loads are out.

  // One tile (block index blk of the launch's tile list).
  auto run_tile = [&](const int blk) {
  int lane = threadIdx.x & 63;
#if DQ8_WIDE_PERSIST > 0
  // the lane id through an empty volatile asm: everything derived from it is
  // recomputed per tile instead of being held in registers across the tiles
  asm volatile("" : "+v"(lane));
#endif
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int pidx = find_proj<true>(b, blk);
  const Proj P = b.p[pidx];
  int mt, nt;
  tile_of(P, blk - P.wave_begin, mt, nt);
  // A SwiGLU pair block covers BN/2 output columns: wave wn's column tile 0
  // is the gate projection's, tile 1 the up projection's, of the same 32
  // outputs (RT == 1, CT == 2 only).
  // The pair mode is compiled into the plain kernels and, with adapters, only
  // into the PL ones (its epilogue would raise every adapter launch's registers).
  constexpr bool CAN_PAIR = !DOTS && wide_pair_shape(WN, RT, CT) && (!LORA || PL);
  const bool pair = CAN_PAIR && P.pair;
  const int m0 = mt * BM, n0 = nt * (pair ? BN / 2 : BN);
  const int G = P.g;
  auto swz = [](int r) { return SWZ == 0 ? (r >> 2) & 3 : (r >> 1) & 3; };

  // 16-byte loads: slot k of this wave is load i = k*NW + wid (A slab i, or B
  // fragment i - AS), landing at frag[i].  Address = uniform base + group *
  // stride (scalar: 64 bytes for an A slab, 2 KB for a B fragment pair) + a
  // fixed lane offset.
  const uint8_t* sbase[L16];
  uint32_t loff[L16];
#pragma unroll
  for (int k = 0; k < L16; ++k) {
    const int i = k * NW + wid;
    if (i < AS) {
      const int rr = lane >> 2;
      const int r0 = min(m0 + 16 * i, P.m - 1);
      const int row = min(m0 + 16 * i + rr, P.m - 1);
      sbase[k] = reinterpret_cast<const uint8_t*>(P.q) + (size_t)r0 * P.ldq;
      loff[k] = (uint32_t)((row - r0) * P.ldq + 16 * ((lane & 3) ^ swz(rr)));
    } else if (pair) {
      // fragment fb: column tile ct = fb/2 of the block is tile ct%2 (gate or
      // up) of wave ct/2, output columns n0 + 32*(ct/2) ..
      const int fb = i - AS, ct = fb >> 1;
      sbase[k] = ((ct & 1) ? P.wt2 : P.wt) + ((size_t)(n0 / 32 + (ct >> 1)) * G * 2 + (fb & 1)) * kFragBytes;
      loff[k] = (uint32_t)lane * 16;
    } else {
      const int fb = i - AS;
      sbase[k] = P.wt + ((size_t)(n0 / 32 + (fb >> 1)) * G * 2 + (fb & 1)) * kFragBytes;
      loff[k] = (uint32_t)lane * 16;
    }
  }
  // w scales: wave w < WSD loads columns 64w .. 64w+63; the others repeat wave
  // w % WSD's load (same data, same place).  Row G of the scales is zero.
  // (SwiGLU pair: wave 0 loads the gate scales of the block's 64 outputs,
  // wave 1 the up scales, to ws[0..63] and ws[64..127].)
  const int ww = WSD > 0 ? wid % (WSD > 0 ? WSD : 1) : 0;
  const float* wsbase = pair ? (ww ? P.wst2 : P.wst) + n0 : P.wst + n0 + 64 * ww;
  const uint32_t wsrow = 4u * (uint32_t)P.np;  // bytes per w-scale row
  // x-scale pieces: load d = k*NW + wid of a chunk covers rows RPD*d .. RPD*d+RPD-1;
  // lane l fetches row l/PPR, piece (l%PPR) ^ (row%PPR).

  // A group's offsets are formed in 32 bits (one scalar add with carry per
  // load): weight handles keep k <= 2^26 and their w-scale table under 4 GiB.
  auto issue_a = [&](AStage& S, int g) {
    const uint32_t gc = (uint32_t)min(g, G - 1);
#pragma unroll
    for (int k = 0; k < KA; ++k) dma16s(sbase[k] + gc * (uint32_t)kGroup, loff[k], &S.frag[k * NW + wid][0]);
  };
  auto issue_b = [&](BStage& S, int g) {
    const uint32_t gc = (uint32_t)min(g, G - 1);
#pragma unroll
    for (int k = KA; k < L16; ++k)
      dma16s(sbase[k] + gc * (uint32_t)(2 * kFragBytes), loff[k], &S.frag[k * NW + wid - AS][0]);
    if constexpr (!DOTS)
      dma4s(reinterpret_cast<const char*>(wsbase) + (uint32_t)min(g, G) * wsrow, (uint32_t)lane * 4, &S.ws[64 * ww]);
  };
  auto issue_x = [&](int c) {  // once per XCH groups: addresses are recomputed here, not kept live
    int ln;  // lane id, read here so that nothing derived from it stays live across the loop
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int xr = ln / PPR, xp = (ln % PPR) ^ (xr % PPR);
    const int g0 = XCH * c + 4 * xp;
    const uint32_t off = 4u * (uint32_t)(g0 < G ? g0 : 0);  // pieces past the last group: in-bounds dummy, never read
#pragma unroll
    for (int k = 0; k < XPW; ++k) {
      const int d = k * NW + wid;
      if (XD % NW == 0 || d < XD) {  // wave-uniform
        const int r0 = min(m0 + RPD * d, P.m - 1);
        const uint32_t row = (uint32_t)((min(m0 + RPD * d + xr, P.m - 1) - r0) * P.ldxs * 4);
        dma16s(P.xs + (size_t)r0 * P.ldxs, row + off, &xc[c & 1].d[d][0]);
      }
    }
  };

  const int wm = wid / WN, wn = wid - (wid / WN) * WN;
  const int fbw = 2 * CT * wn;  // first B fragment of this wave
  // A operand: lane reads row R = WR*wm + 32r + lane%32, chunk 2h + lane/32.
  int aoff[RT][2];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int R = WR * wm + 32 * r + (lane & 31);
      const int rr = R & 15, c = 2 * h + (lane >> 5);
      aoff[r][h] = (R >> 4) * kFragBytes + 16 * (4 * rr + (c ^ swz(rr)));
    }
  // x scale of this lane's K=1 A row: RT == 2: row WR*wm + lane; RT == 1: row WR*wm + lane%32.
  // Its address for group g: (xbx ^ 16*(gg/4)) + 4*(gg%4) + chunk buffer, with
  // gg = g % XCH; xbase has its low 4 + log2(PPR) bits clear, so the XOR only
  // swizzles the piece index.
  const int xrow = WR * wm + (RT == 2 ? lane : (lane & 31));
  const int xbase = (xrow / RPD) * kFragBytes + 16 * ((xrow % RPD) * PPR);
  const int xbx = xbase + 16 * ((xrow % RPD) % PPR);

  v16i cinit;
#pragma unroll
  for (int i = 0; i < 16; ++i) cinit[i] = kMagicBits;
  v32f zero32;
#pragma unroll
  for (int i = 0; i < 32; ++i) zero32[i] = 0.0f;
  v32f s[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) s[j] = zero32;

  // Prologue: A of groups 0 .. SA-2 and B of groups 0 .. SB-2, each A before
  // the B of its group (the order the waits count on).
  if constexpr (!DOTS) issue_x(0);
#pragma unroll
  for (int i = 0; i < SB - 1; ++i) {
    if (i < SA - 1) issue_a(ring.a[i], i);
    issue_b(ring.b[i], i);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (b.unless && *b.unless) {  // uniform: the block leaves once its loads into LDS have landed
    wait_vmcnt<0>();
    return;
  }
  for (int g0 = 0; g0 < G; g0 += PERIOD) {
#pragma unroll
    for (int d = 0; d < PERIOD; ++d) {
      const int g = g0 + d;
      if (g >= G) break;  // uniform over the block
      const AStage& ca = ring.a[d % SA];
      const BStage& cur = ring.b[d % SB];
      wait_vmcnt<WAITN>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // A of group g + SA - 1 and B of group g + SB - 1 go to the slots of
      // group g - 1, which every wave has finished reading (the barrier).
      const int ga = g + SA - 1, gb = g + SB - 1;
      if constexpr (!DOTS) {
        if (ga % XCH == 0 && ga < G) issue_x(ga / XCH);
      }
      issue_a(ring.a[(d + SA - 1) % SA], ga);
      issue_b(ring.b[(d + SB - 1) % SB], gb);
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* fa = &ca.frag[0][0];
      const uint8_t* fr = &cur.frag[0][0];
      v4i af[RT][2], bf[CT][2];
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) af[r][h] = *reinterpret_cast<const v4i*>(fa + aoff[r][h]);
#pragma unroll
      for (int j = 0; j < CT; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          bf[j][h] = *reinterpret_cast<const v4i*>(fr + (fbw + 2 * j + h) * kFragBytes + 16 * lane);
      v16i dt[RT][CT];
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int j = 0; j < CT; ++j) dt[r][j] = mfma_i8(af[r][0], bf[j][0], cinit);
      // cinit stays in its 16 VGPRs: left to itself the compiler rebuilds it
      // from SGPRs in half the groups (8 v_mov_b64 each)
      asm volatile("" : "+v"(cinit));
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
              if (row < P.m && col < P.n) P.dots[((size_t)row * P.n + col) * G + g] = dt[r][j][v] - kMagicBits;
            }
      } else {
        const int gg = g % XCH;
        const int xoff = (xbx ^ (16 * (gg >> 2))) + 4 * (gg & 3) + ((g / XCH) & 1) * (int)sizeof(XChunk);
        const float x = *reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(&xc[0]) + xoff);
#pragma unroll
        for (int j = 0; j < NP; ++j) {
          const v16i& lo = RT == 2 ? dt[0][j] : dt[0][0];
          const v16i& hi = RT == 2 ? dt[1][j] : dt[0][1];
          const float w = RT == 2 ? cur.ws[WC * wn + 32 * j + (lane & 31)]
                          : cur.ws[pair ? 64 * (lane >> 5) + 32 * wn + (lane & 31) : WC * wn + lane];
          const v32f dv = mfma_k1(-kMagic, 1.0f, concat(lo, hi));
          const v32f pv = mfma_k1(x, w, zero32);
          s[j] = s[j] + dv * pv;
        }
      }
    }
  }
  // Drain the clamped loads of the groups past the end before the block exits.
  wait_vmcnt<0>();
  if constexpr (CAN_PAIR) {
    if (pair) {
      // y = s + bias for both projections (tensor.rs:437) and their adapter
      // terms, then the up projection's SwiGlu store over the gate's result
      // (tensor.rs:96-99, qwen.rs:489-490): h = silu(y_gate) * y_up, each op
      // rounded.
      const int mw = m0 + WR * wm, col = n0 + 32 * wn + (lane & 31);
      const float bg = P.bias != nullptr && col < P.n ? P.bias[col] : 0.0f;
      const float bu = P.bias2 != nullptr && col < P.n ? P.bias2[col] : 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s[0][v] = s[0][v] + bg;
        s[0][16 + v] = s[0][16 + v] + bu;
      }
      if constexpr (LORA) {
        // then each projection's adapter term (Adapter::combine, tensor.rs:109-117,
        // after the bias: 438): gate's on column tile 0, up's on tile 1, in this
        // wave's kLoraStage bytes of the idle ring
        static_assert(sizeof(Ring) >= NW * kLoraStage, "adapter staging fits the ring");
        if (P.lora || P.lora2) {
          __builtin_amdgcn_sched_barrier(0);
          lds_barrier();  // every wave is done reading the ring
          float* lw = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(&ring) + wid * kLoraStage);
#pragma unroll
          for (int bk = 0; bk < 2; ++bk) {
            if (bk == 0 ? !P.lora : !P.lora2) continue;  // uniform (lora2 is read with the other pair fields)
            v16f base;
#pragma unroll
            for (int v = 0; v < 16; ++v) base[v] = s[0][16 * bk + v];
            if (bk == 0) {
              base = lora_block32(base, P.lmid, P.lb, P.rank, P.lscale, P.m, P.n, mw, n0 + 32 * wn, lane, lw);
            } else {
              // the up adapter's fields, read here rather than kept in registers
              // across the main loop (the empty asm keeps the loads from moving up)
              int pi = __builtin_amdgcn_readfirstlane(pidx);
              asm volatile("" : "+s"(pi));
              const Proj* pp = &b.p[pi];
              base = lora_block32(base, pp->lmid2, pp->lb2, pp->rank2, pp->lscale2, P.m, P.n, mw, n0 + 32 * wn,
                                  lane, lw);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) s[0][16 * bk + v] = base[v];
            __builtin_amdgcn_sched_barrier(0);  // one adapter block's operands live at a time
          }
        }
      }
      const ExpTab T = exp_table(lane);
      float hv[16];
      // A wave tile inside m x n (uniform) stores with no per-value checks: a
      // wave-uniform row base plus a fixed 32-bit lane offset per store.
      auto h_tile = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        const uint32_t loff = (uint32_t)((4 * (lane >> 5)) * P.n + col) * 4u;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = mw + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const float yg = s[0][v], yu = s[0][16 + v];
          hv[v] = silu_wave(yg, T) * yu;
          if constexpr (FULL) {
            char* rb = reinterpret_cast<char*>(P.out + (size_t)(mw + 8 * (v >> 2) + (v & 3)) * P.n);
            st_out(reinterpret_cast<float*>(rb + loff), hv[v]);
          } else {
            if (row < P.m && col < P.n) st_out(P.out + (size_t)row * P.n + col, hv[v]);
          }
          if ((v & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      };
      if (mw + 32 <= P.m && n0 + 64 <= P.n)
        h_tile(std::true_type{});
      else
        h_tile(std::false_type{});
      if (P.hq != nullptr) {  // uniform over the launch
        // h re-quantized for the down projection (qwen.rs:491, QuantizedInputs::new,
        // tensor.rs:321-339): the block holds 64 whole groups (rows m0.., columns
        // n0 .. n0+63, n0 a multiple of 64).  The tile goes through the idle LDS
        // ring, rows padded to HP floats; then 4 consecutive threads take one
        // row's group, 16 columns each, and compute exactly what k_quantize does.
        constexpr int HP = 72;
        static_assert(BM * HP * 4 <= (int)sizeof(Ring), "h tile fits the ring");
        float* th = reinterpret_cast<float*>(&ring);
        lds_barrier();  // every wave has drained its ring loads and is done reading the ring
#pragma unroll
        for (int v = 0; v < 16; ++v)
          th[(WR * wm + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * HP + 32 * wn + (lane & 31)] = hv[v];
        lds_barrier();
        const int t = threadIdx.x, rl = t >> 2, c0 = 16 * (t & 3);
        const int row = m0 + rl, cb = n0 + c0;
        float e[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v4f f = *reinterpret_cast<const v4f*>(th + rl * HP + c0 + 4 * j);
#pragma unroll
          for (int i = 0; i < 4; ++i) e[4 * j + i] = f[i];
        }
        if (n0 + kGroup > P.n) {  // the last, partial group (uniform): columns past n count as zero, as in k_quantize
#pragma unroll
          for (int i = 0; i < 16; ++i) e[i] = cb + i < P.n ? e[i] : 0.0f;
        }
        // absmax and the finite check from the magnitudes' bit patterns, as in
        // k_quantize_loop (a NaN, only with the flag set, makes the scale NaN)
        uint32_t mb = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) mb = max(mb, __builtin_bit_cast(uint32_t, e[i]) & 0x7fffffffu);
        const bool bad = mb >= 0x7f800000u;
        const float mx = max_quad(__builtin_bit_cast(float, mb));  // the group's 4 threads are lanes 4j .. 4j+3
        const float scale = quant_scale_fma(mx);
        uint32_t w4[4];
        quant_pack<16, true>(e, scale, w4);
        if (row < P.m) {
          int8_t* qr = P.hq + (size_t)row * P.n + cb;
          if ((P.n & 15) == 0 && ((uintptr_t)P.hq & 15) == 0) {
            if (cb < P.n) *reinterpret_cast<uint4*>(qr) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
          } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (cb + i < P.n) qr[i] = (int8_t)(w4[i >> 2] >> (8 * (i & 3)));
          }
          if ((t & 3) == 0) P.hs[(size_t)row * ((P.n + kGroup - 1) / kGroup) + nt] = scale;
        }
        const unsigned long long bb = __ballot(bad && row < P.m);
        if (bb != 0 && lane == __builtin_ffsll((long long)bb) - 1) atomicOr(P.hflag, 1u);
      }
      return;
    }
  }
  if constexpr (!DOTS) {
    const int mw = m0 + WR * wm, nw = n0 + WC * wn;
    // y = s + bias[col], or s + 0.0f without a bias (tensor.rs:437)
    float bias[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int col = nw + 32 * c + (lane & 31);
      bias[c] = P.bias != nullptr && col < P.n ? P.bias[col] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int v = 0; v < 32; ++v) s[j][v] = s[j][v] + bias[RT == 2 ? j : v >> 4];
    if (LORA && P.lora) {
      // then + scale * (mid . b + 0.0) (tensor.rs:438, 109-117), one 32x32
      // block at a time: block b of pair j is row tile b (RT == 2) or column
      // tile b (RT == 1); products from a K=2 MFMA whose k=1 operands (lanes
      // 32-63) are zero.  For rank <= 16 the wave first copies its mid rows and
      // b columns into the (now idle) LDS ring; the products then wait on LDS,
      // not L2.
      v16f zero16;
#pragma unroll
      for (int i = 0; i < 16; ++i) zero16[i] = 0.0f;
      const bool k0 = lane < 32;
      // Operand rows padded to kLoraRow = 17 floats: the 32 lanes reading one
      // element of 32 consecutive rows hit 32 banks, and every operand read is
      // a base register plus an immediate offset (no address arithmetic).
      constexpr int WROWS = 32 * RT, WCOLS = 32 * CT, LWAVE = (WROWS + WCOLS) * kLoraRow * 4;
      constexpr bool FITS = NW * LWAVE <= (int)sizeof(Ring);
      const bool staged = FITS && P.rank <= 16;
      float* lmid = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(&ring) + wid * LWAVE);
      float* lbw = lmid + WROWS * kLoraRow;
      auto sw = [](int r, int i) { return r * kLoraRow + i; };
      if (staged) {
        lds_barrier();  // every wave is done reading the ring
        // The wave's mid rows mw.. and b rows nw.. are contiguous runs of
        // WROWS * rank and WCOLS * rank floats: the lanes load them together
        // (each load instruction covers whole cache lines), all loads first,
        // then the LDS writes.  Rows past m or n read the last row instead.
        static_assert(WROWS <= 64 && WCOLS <= 64, "at most 64 rows and columns per wave");
        const int rk = P.rank;
        if (rk == 16 && ((size_t)P.lmid & 15) == 0 && ((size_t)P.lb & 15) == 0) {
          constexpr int TM = WROWS / 16, TB = WCOLS / 16;  // float4 per lane
          v4f vm[TM], vb[TB];
#pragma unroll
          for (int t = 0; t < TM; ++t) {
            const int e = 64 * t + lane;  // float4 index: row e/4, inputs 4(e%4)..+3
            vm[t] = *reinterpret_cast<const v4f*>(P.lmid + (size_t)min(mw + (e >> 2), P.m - 1) * 16 + 4 * (e & 3));
          }
#pragma unroll
          for (int t = 0; t < TB; ++t) {
            const int e = 64 * t + lane;
            vb[t] = *reinterpret_cast<const v4f*>(P.lb + (size_t)min(nw + (e >> 2), P.n - 1) * 16 + 4 * (e & 3));
          }
#pragma unroll
          for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = 64 * t + lane;
              lmid[sw(e >> 2, 4 * (e & 3) + q)] = vm[t][q];
            }
#pragma unroll
          for (int t = 0; t < TB; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = 64 * t + lane;
              lbw[sw(e >> 2, 4 * (e & 3) + q)] = vb[t][q];
            }
        } else {
          // element e of a run is row e / rank, input e % rank; with e < 1024
          // and rank <= 16, (e + 0.5) / rank lies at least 1/32 from an integer,
          // so the float quotient truncates to the exact row
          const float inv = 1.0f / (float)rk;
          auto row_of = [&](int e) { return (int)(((float)e + 0.5f) * inv); };
          float vm[WROWS / 4], vb[WCOLS / 4];  // up to 16 * rows / 64 floats per lane
#pragma unroll
          for (int t = 0; t < WROWS / 4; ++t) {
            const int e = 64 * t + lane, row = row_of(e);
            vm[t] = row < WROWS ? P.lmid[(size_t)min(mw + row, P.m - 1) * rk + (e - row * rk)] : 0.0f;
          }
#pragma unroll
          for (int t = 0; t < WCOLS / 4; ++t) {
            const int e = 64 * t + lane, row = row_of(e);
            vb[t] = row < WCOLS ? P.lb[(size_t)min(nw + row, P.n - 1) * rk + (e - row * rk)] : 0.0f;
          }
#pragma unroll
          for (int t = 0; t < WROWS / 4; ++t) {
            const int e = 64 * t + lane, row = row_of(e);
            if (row < WROWS) lmid[sw(row, e - row * rk)] = vm[t];
          }
#pragma unroll
          for (int t = 0; t < WCOLS / 4; ++t) {
            const int e = 64 * t + lane, row = row_of(e);
            if (row < WCOLS) lbw[sw(row, e - row * rk)] = vb[t];
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's copies are visible to it
      }
#pragma unroll
      for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int bk = 0; bk < 2; ++bk) {
          const int r = (RT == 2 ? 32 * bk : 0) + (lane & 31);
          const int c = (RT == 2 ? 32 * j : 32 * bk) + (lane & 31);
          v16f base;
#pragma unroll
          for (int v = 0; v < 16; ++v) base[v] = s[j][16 * bk + v];
          if (staged) {
            // The block splits into 4 slices of 4 rows (8u + 4(l/32) + 0..3 for
            // lane l, elements 4u..4u+3 of the block): one
            // v_mfma_f32_4x4x1_16b_f32 forms a slice's products for one index,
            // A lane l = mid[row 8u + 4(l/32) + l%4], B lane l = b[col l%32],
            // so every slice sums on its own in 4 registers.
            // row 8u + 4(l/32) + l%4 of slice u sits 8u rows past slice 0's
            const float* rm0 = lmid + kLoraRow * ((RT == 2 ? 32 * bk : 0) + 4 * (lane >> 5) + (lane & 3));
            const float* rb = lbw + kLoraRow * c;
            const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
            v16f sum;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float* rmu = rm0 + 8 * kLoraRow * u;
              auto prod = [&](int i) { return mfma_k1_4(rmu[i], rb[i], zero4); };
              v4f su;
              if (P.rank == 16) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                  const v4f ln = prod(i) + prod(8 + i);
                  su = i == 0 ? ln : su + ln;
                }
              } else {
                // rank < 16: the lane sums are the products themselves, then
                // the tail, all in index order from the first product
                su = zero4;
                for (int i = 0; i < P.rank; ++i) su = i == 0 ? prod(0) : su + prod(i);
              }
#pragma unroll
              for (int v = 0; v < 4; ++v) sum[4 * u + v] = su[v];
            }
            base = base + P.lscale * (sum + zero16);
          } else {
            const float* lm = P.lmid + (size_t)min(mw + r, P.m - 1) * P.rank;
            const float* lbc = P.lb + (size_t)min(nw + c, P.n - 1) * P.rank;
            base = lora_term(base, zero16, P.rank, P.lscale,
                             [&](int i) { return mfma_k2(k0 ? lm[i] : 0.0f, k0 ? lbc[i] : 0.0f, zero16); });
          }
#pragma unroll
          for (int v = 0; v < 16; ++v) s[j][16 * bk + v] = base[v];
        }
    }
    constexpr int E = NP * 32;
    int rows[E], cols[E];
    float y[E];
    // with the wave's tile inside m x n (uniform), rows and columns split into
    // a wave-uniform part and the lane's fixed offset (4*(lane/32), lane%32)
    const bool full = P.layout == 0 && mw + WR <= P.m && nw + WC <= P.n;
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int v = 0; v < 32; ++v) {
        const int blk2 = v >> 4, vv = v & 15;
        const int r = RT == 2 ? blk2 : 0, c = RT == 2 ? j : blk2;
        rows[32 * j + v] = mw + 32 * r + 8 * (vv >> 2) + (vv & 3) + (full ? 0 : 4 * (lane >> 5));
        cols[32 * j + v] = nw + 32 * c + (full ? 0 : (lane & 31));
        y[32 * j + v] = s[j][v];
      }
    if (full)
      store_tile_full(P, rows, cols, (uint32_t)(4 * (lane >> 5) * P.n + (lane & 31)) * 4u, y);
    else
      store_tile(P, rows, cols, y);
  }
  };
#if DQ8_WIDE_PERSIST > 0
  // A grid of resident blocks walks the tile list: block i takes tiles i, i +
  // gridDim.x, ...  (gridDim.x a multiple of 8 keeps each tile on the XCD the
  // plain launch would give it).  The barrier keeps the next tile's loads out
  // of LDS the previous epilogue may still read.
  for (int t = blockIdx.x; t < b.total_waves; t += gridDim.x) {
    run_tile(t);
    __syncthreads();
  }
#else
  run_tile(blockIdx.x);
#endif
}

// ---------------------------------------------------------------------------
// Skinny projection kernel (M <= 32).  Per group and 16 x 16 tile:
//   v_mfma_i32_16x16x64_i8 gives the group's dots (lane l, element v: row
//   4*(l/16) + v, column l%16), C = the bias bits 0x4B400000;
//   v_mfma_f32_4x4x1_16b_f32 with A = -12582912, B = 1 converts them exactly;
//   the same instruction with A lane a = x of row 4*(a/16) + a%4 and B lane l =
//   w of column l%16 is the product outer product in the same layout.
//
// The kernel is a weight stream.  Its speed is set by the weight bytes in
// flight (HBM latency under load is microseconds), so every wave keeps a deep
// register ring of weight fragments and w scales, and a wave covers all rows
// of its strip of 16*CT columns (each weight byte is loaded once):
//  * short K (G <= 32): the block first loads its whole activation (16*RT rows
//    x G*64 bytes, at most 64 KB) and x scales into LDS; then the waves run
//    with no barriers.  Activation bytes land by direct loads of 8 rows x 128
//    bytes (two groups; 8 whole cache lines per load): lane l fetches row l/8,
//    16-byte chunk (l%8) ^ (l/8) and lands at slot l, so the MFMA operand
//    reads are free of bank conflicts.
//  * long K (G > 32): a strip's groups are interleaved over NSEG = 4 waves
//    (wave sidx takes the groups g with g % NSEG == sidx), so a strip has
//    NSEG rings in flight.  A block covers one 16-row tile of its strip (17-32
//    rows: two blocks per strip, so each weight byte is read twice, the second
//    time mostly from cache), so a ring step is one activation and one weight
//    fragment and the ring runs 6 steps ahead (the load latency under a full
//    stream is microseconds; 8 steps measured 1-2% slower for a 24-row layer
//    set at 180 against 144 VGPRs).  Activation fragments join the register ring;
//    x scales come through LDS in chunks of 8 steps.  Per step every wave
//    posts its t's to LDS and, after a barrier, the strip's first wave adds
//    them in group order: every output is still one left-to-right sum.
// x scales in LDS: [row][piece of 4 groups] in 16-byte pieces, loaded 64
// pieces per direct load (lane l: row l/XP, piece (l%XP) ^ (row%XP), XP pieces
// per row) and read back with the same XOR.  Rows past M repeat row M-1 and
// loads past the last group repeat the last one: every load stays in bounds;
// no output of such a row or group is stored.
__device__ __forceinline__ v4i mfma_i8_16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// LDS bytes of the skinny kernel: the short-K preload (16 steps of activation
// plus 32 groups of x scales) or the long-K x chunks and posted t's (ctl
// column tiles per long-K wave).
constexpr int skinny_lds_bytes(int rt, int ctl) {
  const int short_k = 16 * rt * 2 * kFragBytes + 16 * rt * 8 * 16;
  const int long_k = 2 * 16 * rt * 8 * 16 + 2 * 4 * rt * ctl * kFragBytes;
  return short_k > long_k ? short_k : long_k;
}

// Byte offset in an x chunk of XP pieces per row of (row r, group gg of the chunk).
template <int XP>
__device__ __forceinline__ int x_slot(int r, int gg) {
  return 16 * (r * XP + ((gg >> 2) ^ (r % XP))) + 4 * (gg & 3);
}

// Direct loads of x chunk c (XP pieces of 4 groups per row, ROWS rows from row
// r0) into dst: this wave's share of the ROWS*XP/64 loads.  Needs 16-byte
// aligned rows of ldxs % 4 == 0 floats.
template <int ROWS, int XP>
__device__ __forceinline__ void issue_x_chunk(const Proj& P, int c, int wid, uint8_t* dst, int r0 = 0) {
  constexpr int LOADS = (ROWS * XP + 63) / 64;
  const int last_piece = (P.g + 3) / 4 - 1;
  int ln;  // lane id, read here so that nothing derived from it stays live
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
  for (int k = 0; k < (LOADS + 3) / 4; ++k) {
    const int i = wid + 4 * k;
    if (i < LOADS) {
      const int e = 64 * i + ln;
      const int r = e / XP, pc = (e % XP) ^ (r % XP);
      const int gp = min(c * XP + pc, last_piece);
      const uint32_t off = (uint32_t)(min(r0 + r, P.m - 1) * P.ldxs + 4 * gp) * 4u;
      dma16s(P.xs, off, dst + i * kFragBytes);
    }
  }
}

// y = s + bias, or s + 0.0f without a bias (tensor.rs:437), then the LoRA term
// (tensor.rs:438, 109-117) when the projection has an adapter, stored by the
// epilogue.  LoRA products: K=1 MFMA with A lane a = mid of row 4*(a/16) + a%4
// and B lane l = b of column l%16, the x/w scale convention of the group loop.
template <int RT, int CT, bool LORA>
__device__ __forceinline__ void skinny_store(const Proj& P, int c0, int lane, v4f (&s)[RT * CT], int r0 = 0) {
  constexpr int E = 4 * RT * CT;
  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int col = c0 + 16 * ct + (lane & 15);
    const float bias = P.bias != nullptr && col < P.n ? P.bias[col] : 0.0f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) s[rt * CT + ct] = s[rt * CT + ct] + bias;
  }
  if (LORA && P.lora) {
    const float* lm[RT];
    const float* lbc[CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      lm[rt] = P.lmid + (size_t)min(r0 + 16 * rt + 4 * (lane >> 4) + (lane & 3), P.m - 1) * P.rank;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) lbc[ct] = P.lb + (size_t)min(c0 + 16 * ct + (lane & 15), P.n - 1) * P.rank;
    if (P.rank <= 16) {
      // every operand of the strip loaded up front (one memory latency), as
      // 16-byte loads when rank is 16 and the rows are 16-byte aligned
      float am[RT][16], bm[CT][16];
      if (P.rank == 16 && ((size_t)P.lmid & 15) == 0 && ((size_t)P.lb & 15) == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const v4f v = *reinterpret_cast<const v4f*>(lm[rt] + 4 * q);
#pragma unroll
            for (int u = 0; u < 4; ++u) am[rt][4 * q + u] = v[u];
          }
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            const v4f v = *reinterpret_cast<const v4f*>(lbc[ct] + 4 * q);
#pragma unroll
            for (int u = 0; u < 4; ++u) bm[ct][4 * q + u] = v[u];
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) am[rt][i] = i < P.rank ? lm[rt][i] : 0.0f;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) bm[ct][i] = i < P.rank ? lbc[ct][i] : 0.0f;
        }
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          s[rt * CT + ct] = lora_term16(s[rt * CT + ct], zero4, P.rank, P.lscale,
                                        [&](int i) { return mfma_k1_4(am[rt][i], bm[ct][i], zero4); });
    } else {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          s[rt * CT + ct] = lora_term(s[rt * CT + ct], zero4, P.rank, P.lscale,
                                      [&](int i) { return mfma_k1_4(lm[rt][i], lbc[ct][i], zero4); });
    }
  }
  int rows[E], cols[E];
  float y[E];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int e = 4 * (rt * CT + ct) + v;
        rows[e] = r0 + 16 * rt + 4 * (lane >> 4) + v;
        cols[e] = c0 + 16 * ct + (lane & 15);
        y[e] = s[rt * CT + ct][v];
      }
  store_tile(P, rows, cols, y);
}

// One group of a wave's tiles: dots (exported when DOTS) or t = dot * p.
template <int RT, int CT, bool DOTS>
__device__ __forceinline__ void skinny_group(const Proj& P, int c0, int lane, bool store, int g, const v4i (&a)[RT],
                                             const v4i (&bw)[CT], const float (&x)[RT], const float (&ws)[CT],
                                             v4f (&t)[RT * CT], int r0 = 0) {
  const v4i magic = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const v4i dd = mfma_i8_16(a[rt], bw[ct], magic);
      if constexpr (DOTS) {
        if (store) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = r0 + 16 * rt + 4 * (lane >> 4) + v;
            const int col = c0 + 16 * ct + (lane & 15);
            if (row < P.m && col < P.n) P.dots[((size_t)row * P.n + col) * P.g + g] = dd[v] - kMagicBits;
          }
        }
      } else {
        const v4f dv = mfma_k1_4(-kMagic, 1.0f, __builtin_bit_cast(v4f, dd));
        const v4f pv = mfma_k1_4(x[rt], ws[ct], zero4);
        t[rt * CT + ct] = dv * pv;
      }
    }
}

// 1: the short-K weight loads are non-temporal: each weight byte is read once,
// and the stream no longer displaces the activations and the long-K weights
// that the other blocks re-read from L2 (24-row layer set: 18.5 -> 17.2 us per
// question launch).  Non-temporal w-scale loads measured no better, and
// non-temporal long-K weight loads slower (both row-tile blocks of a strip
// read them).
#ifndef DQ8_SKINNY_NT_SHORT
#define DQ8_SKINNY_NT_SHORT 1
#endif
// Short K (G <= 32): one wave streams the 16*CT columns from c0 over all
// groups, 2 groups per step.  The block's 4 waves first load its activation
// together; a wave with no columns (live false) only helps with that.
template <int RT, int CT, int DB, bool DOTS, bool LORA>
__device__ __forceinline__ void skinny_short(const Proj& P, int c0, bool live, int wid, int lane, uint8_t* lds,
                                             const uint32_t* unless) {
  constexpr int ROWS = 16 * RT;
  constexpr int STEP_A = RT * 2 * kFragBytes;  // activation bytes of one step (8-row units)
  constexpr int OPS = 2 * CT * (DOTS ? 1 : 2);  // ring loads per step
  static_assert(DB >= 2 && (DB - 1) * OPS <= 63, "ring depth");
  uint8_t* xl = lds + 16 * STEP_A;  // x scales: one chunk of 32 groups (8 pieces per row)
  const int G = P.g;
  const int steps = (G + 1) >> 1;

  const uint8_t* pb[CT];
  const float* pw[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int cc = c0 + 16 * ct;
    pb[ct] = P.wt + ((size_t)(cc >> 5) * G * 2 + (lane >> 5)) * kFragBytes +
             ((cc & 31) + (lane & 15) + 32 * ((lane >> 4) & 1)) * 16;
    pw[ct] = P.wst + cc + (lane & 15);
  }
  v4i bq[DB][2][CT];
  float wq[DB][2][CT];
  auto issue = [&](v4i (&bs)[2][CT], float (&ws)[2][CT], int j) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int g = min(2 * j + gi, G - 1);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#if DQ8_SKINNY_NT_SHORT
        bs[gi][ct] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(pb[ct] + (size_t)g * 2 * kFragBytes));
#else
        bs[gi][ct] = load16(pb[ct] + (size_t)g * 2 * kFragBytes);
#endif
        if constexpr (!DOTS) ws[gi][ct] = pw[ct][(size_t)g * P.np];
      }
    }
  };
  if (live) {
#pragma unroll
    for (int d = 0; d < DB - 1; ++d) {
      issue(bq[d], wq[d], min(d, steps - 1));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Preload: activation unit u = 2*RT*j + o (step j, row octet o), then the x chunk.
  {
    const int units = steps * 2 * RT;
    const int sr = lane >> 3, c8 = (lane & 7) ^ (lane >> 3);
    for (int u = wid; u < units; u += 4) {
      const int j = u / (2 * RT), o = u - j * 2 * RT;
      const int grp = min(2 * j + (c8 >> 2), G - 1);
      const uint32_t off = (uint32_t)(min(8 * o + sr, P.m - 1) * P.ldq + 64 * grp + 16 * (c8 & 3));
      dma16s(P.q, off, lds + j * STEP_A + o * kFragBytes);
    }
    if constexpr (!DOTS) issue_x_chunk<ROWS, 8>(P, 0, wid, xl);
  }
  // the non-finite flag is read while the first loads are in flight; the
  // whole block leaves on it (after they land: they write this block's LDS)
  const bool skip = unless != nullptr && *unless != 0;
  wait_vmcnt<0>();
  if (skip) return;
  lds_barrier();
  if (!live) return;  // no later barrier in this path

  int aoff[RT][2];  // [row tile][group parity]: row 16rt + l%16, chunk 4*parity + l/16
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int r = 16 * rt + (lane & 15), c8 = 4 * par + (lane >> 4);
      aoff[rt][par] = (r >> 3) * kFragBytes + 16 * (8 * (r & 7) + (c8 ^ (r & 7)));
    }
  int xr[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) xr[rt] = 16 * rt + 4 * (lane >> 4) + (lane & 3);

  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  v4f s[RT * CT];
#pragma unroll
  for (int k = 0; k < RT * CT; ++k) s[k] = zero4;
  // Step j from ring slot d (a constant after unrolling).  Every slot is
  // consumed on every path (the odd last group is computed on a clamped copy
  // and dropped), and the ring loop has no early exit: the compiler's load
  // waits then stay exact instead of draining the ring at the loop header.
  auto step = [&](int j, int d) __attribute__((always_inline)) {
    const int nd = (d + DB - 1) % DB;
    issue(bq[nd], wq[nd], min(j + DB - 1, steps - 1));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int g = 2 * j + gi;
      const int gx = min(g, G - 1);
      v4i a[RT];
      float x[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        a[rt] = *reinterpret_cast<const v4i*>(lds + j * STEP_A + aoff[rt][gi]);
        if constexpr (!DOTS) x[rt] = *reinterpret_cast<const float*>(xl + x_slot<8>(xr[rt], gx));
      }
      v4f t[RT * CT];
      skinny_group<RT, CT, DOTS>(P, c0, lane, live && g < G, g, a, bq[d][gi], x, wq[d][gi], t);
      if constexpr (!DOTS) {
        if (g < G) {  // uniform
#pragma unroll
          for (int k = 0; k < RT * CT; ++k) s[k] = s[k] + t[k];
        }
      }
    }
  };
  int j0 = 0;
  for (; j0 + DB <= steps; j0 += DB) {
#pragma unroll
    for (int d = 0; d < DB; ++d) step(j0 + d, d);
  }
#pragma unroll
  for (int d = 0; d < DB - 1; ++d)
    if (j0 + d < steps) step(j0 + d, d);
  wait_vmcnt<0>();  // the clamped loads past the end
  if constexpr (!DOTS)
    if (live) skinny_store<RT, CT, LORA>(P, c0, lane, s);
}

// Long K (G > 32): one strip per block (TPB = 4/NSEG = 1), its 16*RT rows from row
// r0, NSEG waves, one group per wave and step.
template <int RT, int CT, int DB, int NSEG, bool DOTS, bool LORA>
__device__ __forceinline__ void skinny_long(const Proj& P, int local, int wid, int lane, uint8_t* lds, int r0,
                                            const uint32_t* unless) {
  constexpr int ROWS = 16 * RT, NT = RT * CT, TPB = 4 / NSEG;
  constexpr int XP = 2 * NSEG;                 // x pieces per row of a chunk of 8 steps (8*NSEG groups)
  constexpr int XBYTES = ROWS * XP * 16;
  constexpr int OPS = CT * (DOTS ? 1 : 2) + RT;  // ring loads per step
  static_assert(DB >= 2 && (DB - 1) * OPS <= 63 && DB <= 10, "ring depth");
  constexpr int WAIT_X0 = (DB - 1) * OPS, WAIT_X = 8 * OPS < 63 ? 8 * OPS : 63;
  uint8_t* xl = lds;  // x chunks, double-buffered
  v4f(*tb)[4][NT][64] = reinterpret_cast<v4f(*)[4][NT][64]>(lds + 2 * XBYTES);  // posted t's
  const int sidx = wid % NSEG, tib = wid / NSEG;
  const int strip = local * TPB + tib;
  const bool live = strip < P.waves_n;
  const int c0 = (live ? strip : 0) * 16 * CT;
  const int G = P.g;
  const int steps = (G + NSEG - 1) / NSEG;
  const int chunks = (G + 8 * NSEG - 1) / (8 * NSEG);

  const int8_t* pa[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) pa[rt] = P.q + (size_t)min(r0 + 16 * rt + (lane & 15), P.m - 1) * P.ldq + 16 * (lane >> 4);
  const uint8_t* pb[CT];
  const float* pw[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int cc = c0 + 16 * ct;
    pb[ct] = P.wt + ((size_t)(cc >> 5) * G * 2 + (lane >> 5)) * kFragBytes +
             ((cc & 31) + (lane & 15) + 32 * ((lane >> 4) & 1)) * 16;
    pw[ct] = P.wst + cc + (lane & 15);
  }
  v4i aq[DB][RT], bq[DB][CT];
  float wq[DB][CT];
  auto issue = [&](v4i (&as)[RT], v4i (&bs)[CT], float (&ws)[CT], int j) {
    const int g = min(j * NSEG + sidx, G - 1);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      bs[ct] = load16(pb[ct] + (size_t)g * 2 * kFragBytes);
      if constexpr (!DOTS) ws[ct] = pw[ct][(size_t)g * P.np];
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) as[rt] = load16(pa[rt] + g * kGroup);
  };
  int xr[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) xr[rt] = 16 * rt + 4 * (lane >> 4) + (lane & 3);
  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  v4f s[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) s[k] = zero4;
  auto add_posted = [&](int j) {  // first wave of a strip: the step's t's in group order
    if (sidx == 0) {
      v4f tp[NSEG][NT];  // all reads first, then the adds in order
#pragma unroll
      for (int i = 0; i < NSEG; ++i)
#pragma unroll
        for (int k = 0; k < NT; ++k) tp[i][k] = tb[j & 1][tib * NSEG + i][k][lane];
#pragma unroll
      for (int i = 0; i < NSEG; ++i)
        if (j * NSEG + i < G) {  // uniform: groups past G in the last step are not added
#pragma unroll
          for (int k = 0; k < NT; ++k) s[k] = s[k] + tp[i][k];
        }
    }
  };

  if constexpr (!DOTS) issue_x_chunk<ROWS, XP>(P, 0, wid, xl, r0);
#pragma unroll
  for (int d = 0; d < DB - 1; ++d) {
    issue(aq[d], bq[d], wq[d], min(d, steps - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
  // the non-finite flag, read while the first loads are in flight (the block
  // leaves after they land: the x chunk writes this block's LDS)
  if (unless != nullptr && *unless != 0) {
    wait_vmcnt<0>();
    return;
  }
  // Step j from ring slot d (a constant after unrolling); as in the short-K
  // loop, every slot is consumed on every path and the ring loop has no early
  // exit.  Groups past G (the last step) are computed on clamped copies; their
  // t's are posted but not added.
  auto step = [&](int j, int d) __attribute__((always_inline)) {
    const bool chunk_start = (j & 7) == 0;
    // x chunk j/8 was issued 8 steps ago (chunk 0: before the prologue); the
    // waits let through only the ring loads issued after it.
    if constexpr (!DOTS) {
      if (chunk_start) {
        if (j == 0) wait_vmcnt<WAIT_X0>();
        else wait_vmcnt<WAIT_X>();
      }
    }
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!DOTS) {
      if (chunk_start && (j >> 3) + 1 < chunks)
        issue_x_chunk<ROWS, XP>(P, (j >> 3) + 1, wid, xl + (((j >> 3) + 1) & 1) * XBYTES, r0);
    }
    const int nd = (d + DB - 1) % DB;
    issue(aq[nd], bq[nd], wq[nd], min(j + DB - 1, steps - 1));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!DOTS)
      if (j > 0) add_posted(j - 1);
    const int g = j * NSEG + sidx;
    float x[RT];
    if constexpr (!DOTS) {
      const uint8_t* xc = xl + ((j >> 3) & 1) * XBYTES;
      const int gg = min(g, G - 1) - (j >> 3) * 8 * NSEG;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) x[rt] = *reinterpret_cast<const float*>(xc + x_slot<XP>(xr[rt], gg));
    }
    v4f t[NT];
    skinny_group<RT, CT, DOTS>(P, c0, lane, live && g < G, g, aq[d], bq[d], x, wq[d], t, r0);
    if constexpr (!DOTS) {
#pragma unroll
      for (int k = 0; k < NT; ++k) tb[j & 1][wid][k][lane] = t[k];
    }
  };
  int j0 = 0;
  for (; j0 + DB <= steps; j0 += DB) {
#pragma unroll
    for (int d = 0; d < DB; ++d) step(j0 + d, d);
  }
#pragma unroll
  for (int d = 0; d < DB - 1; ++d)
    if (j0 + d < steps) step(j0 + d, d);
  if constexpr (!DOTS) {
    lds_barrier();
    add_posted(steps - 1);
  }
  wait_vmcnt<0>();  // the clamped loads past the end
  if constexpr (!DOTS)
    if (live && sidx == 0) skinny_store<RT, CT, LORA>(P, c0, lane, s, r0);
}

template <int RT, int CT, int CTL, int DBS, int DBL, bool DOTS, bool LORA>
__global__ __launch_bounds__(256) void k_linear_skinny(Batch b) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[skinny_lds_bytes(RT, CTL)];
  // non-finite inputs (*b.unless != 0): the FP32 kernel runs instead; each
  // path checks the flag once its first loads are out
  const int pidx = find_proj<true>(b, blockIdx.x);
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const Proj P = b.p[pidx];  // by value: its fields load in one batch
  const int local = blockIdx.x - P.wave_begin;
  if (P.nseg == 1) {
    static_assert(CT == 2, "short-K waves take at most two 16-column units");
    const int H = P.waves_n;  // units of 16 columns
    int u0, cnt;
    if (P.units == 8) {
      // 4 strips of two units per block, one per wave, from unit 8*local
      u0 = 2 * (4 * local + wid);
      cnt = u0 < H ? 2 : 0;
    } else {
      // The units are dealt to B = ceil(H / units) blocks, deal_q to each and
      // one more to the first deal_r (at most 7; the host divides), so blocks
      // carry equal byte counts to within one unit, and a block's c units to
      // its waves as evenly as they go (w*c/4 .. (w+1)*c/4): as many waves
      // stream as the block has units, up to 4, and none takes more than two.
      const int h0 = local * P.deal_q + min(local, P.deal_r), c = P.deal_q + (local < P.deal_r ? 1 : 0);
      u0 = h0 + wid * c / 4;
      cnt = h0 + (wid + 1) * c / 4 - u0;
    }
    if (cnt == 2)
      skinny_short<RT, 2, DBS, DOTS, LORA>(P, 16 * u0, true, wid, lane, lds, b.unless);
    else
      skinny_short<RT, 1, DBS, DOTS, LORA>(P, 16 * u0, cnt == 1, wid, lane, lds, b.unless);
  } else if (RT == 1) {
    skinny_long<1, CTL, DBL, 4, DOTS, LORA>(P, local, wid, lane, lds, 0, b.unless);
  } else {
    // One 16-row tile per block: 17-32 rows take two blocks per strip.  The
    // two blocks of a strip are 8 apart (blocks are dealt to the 8 XCDs in
    // turn), so both run on one XCD and the second read of the strip's weights
    // is served by that XCD's L2: in each run of 16 blocks, blocks 0-7 take
    // the first row tile of 8 strips and blocks 8-15 the second.  A last run
    // of R < 8 strips pairs blocks R apart.
    const int run = local >> 4, in = local & 15;
    const int left = P.waves_n - 8 * run;  // strips from this run on
    const int r = left >= 8 ? 8 : left;
    const int t = r == 8 ? in >> 3 : in / r;  // the row tile (a division only in the last run)
    skinny_long<1, CTL, DBL, 4, DOTS, LORA>(P, 8 * run + in - t * r, wid, lane, lds, 16 * t, b.unless);
  }
}
// LoRA middle product (weights.rs:480, 495): mid[r][j] = dot_scores(x_r, a_j)
// + 0.0 for x [m][k], a [rank][k], in dot_scores' x86-64 order (tensor.rs:6-25).
// Two kernels compute it in that order.  k_lora_mid_rows reads plain memory and
// takes any shape and alignment; k_lora_mid_dma (below) stages tiles through
// LDS and needs 16-byte aligned rows.
//
// k_lora_mid_rows:
// A wave covers 4 rows and 8 columns j: lane l works on column j0 + l/8 and
// holds lane i = l%8 of its partial sums (elements i, i+8, ...) for the 4 rows.
// The 8 partial sums are then added in order, the tail elements one by one.
__global__ __launch_bounds__(256) void k_lora_mid_rows(const float* __restrict__ x, int m, int k, const float* __restrict__ a,
                                                  int rank, float* __restrict__ mid) {
  const int lane = threadIdx.x & 63;
  const long wave = (long)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int jblocks = (rank + 7) >> 3;
  if (wave >= (long)((m + 3) >> 2) * jblocks) return;  // wave-uniform
  const int r0 = (int)(wave / jblocks) * 4;
  const int j = (int)(wave % jblocks) * 8 + (lane >> 3), i = lane & 7;
  const float* arow = a + (size_t)min(j, rank - 1) * k;
  const float* xr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) xr[r] = x + (size_t)min(r0 + r, m - 1) * k;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int chunks = k >> 3;
  // Groups of 8 chunks, double-buffered: the loads of the next group are in
  // flight while the current one is added in order.
  struct Grp {
    float av[8], xv[4][8];
  };
  auto load = [&](Grp& g, int c) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      g.av[u] = arow[8 * (c + u) + i];
#pragma unroll
      for (int r = 0; r < 4; ++r) g.xv[r][u] = xr[r][8 * (c + u) + i];
    }
  };
  auto add = [&](const Grp& g) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = acc[r] + g.xv[r][u] * g.av[u];
  };
  int c = 0;
  if (chunks >= 8) {
    Grp g0, g1;
    load(g0, 0);
    c = 8;
    while (true) {
      if (c + 8 > chunks) { add(g0); break; }
      load(g1, c);
      c += 8;
      add(g0);
      if (c + 8 > chunks) { add(g1); break; }
      load(g0, c);
      c += 8;
      add(g1);
    }
  }
  for (; c < chunks; ++c) {
    const float av = arow[8 * c + i];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = acc[r] + xr[r][8 * c + i] * av;
  }
  float sum[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float t = -0.0f;
#pragma unroll
    for (int ii = 0; ii < 8; ++ii) t = t + __shfl(acc[r], (lane & ~7) + ii);
    sum[r] = t;
  }
  for (int t = 8 * chunks; t < k; ++t) {
    const float av = arow[t];
#pragma unroll
    for (int r = 0; r < 4; ++r) sum[r] = sum[r] + xr[r][t] * av;
  }
  if (i == 0 && j < rank) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (r0 + r < m) mid[(size_t)(r0 + r) * rank + j] = sum[r] + 0.0f;
  }
}

// k_lora_mid_dma: a block of 4 waves covers 8 rows of x and 16 adapter rows.
// Tiles of 256 inputs (8 x rows and 16 A rows, 1 KB each) reach LDS by direct
// global->LDS loads in a ring of kMidSlots tiles, kMidSlots - 1 of them in
// flight; wave w loads x rows 2w, 2w+1 and A rows 4w..4w+3 of every tile.
// The products come from v_mfma_f32_4x4x1_16b_f32 with C = +0.0: each output
// is one product rounded once, as a multiply (a zero product may lose its
// sign, which no lane sum can see: a lane sum starts at +0.0, so it is never
// -0.0, and s + 0.0 == s + -0.0 for every other s).  The VALU only adds.
// Block b = 8g + i of the instruction holds lane sum i of rows 4g..4g+3 and
// adapter rows 4w..4w+3 of this wave: A lane l = x[4(l/32) + l%4][8c + (l/4)%8],
// B lane l = A[4w + l%4][8c + (l/4)%8], and output register r of lane l is the
// product for row 4(l/32) + r, adapter row 4w + l%4, lane sum (l/4)%8.  The 8
// lane sums of (row, adapter row) then sit in lanes (l & 32) + 4i + (l & 3);
// they are added in order from -0.0, then the tail elements one by one.
// Loads past the full chunks of 8 are clamped to the row's last 16 bytes and
// never summed.  The row stride of 264 floats keeps the 32 distinct A inputs a
// wave reads per chunk in distinct banks.
// Requires k % 4 == 0 and 16-byte aligned x and a.
constexpr int kMidRows = 8, kMidJ = 16, kMidKT = 256, kMidStride = kMidKT + 8;
#ifndef DQ8_MID_SLOTS
#define DQ8_MID_SLOTS 3
#endif
#ifndef DQ8_MID_BATCH
#define DQ8_MID_BATCH 8
#endif
#ifndef DQ8_MID_PIPE
#define DQ8_MID_PIPE 1
#endif
#ifndef DQ8_MID_SMALL_M
#define DQ8_MID_SMALL_M 32  // rows up to which k_lora_mid_small runs (0: never)
#endif
constexpr int kMidSlots = DQ8_MID_SLOTS, kMidLoads = 6;  // DMA loads per wave per tile
constexpr int kMidBatch = DQ8_MID_BATCH;
typedef float MidTile[kMidSlots][kMidRows + kMidJ][kMidStride];
__device__ __forceinline__ void lora_mid_tiled(const float* __restrict__ x, int m, int k, const float* __restrict__ a,
                                               int rank, float* __restrict__ mid, int block, MidTile& lds) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int jblocks = (rank + kMidJ - 1) / kMidJ;
  const int r0 = (block / jblocks) * kMidRows, j0 = (block % jblocks) * kMidJ;
  const int chunks = k >> 3, full = 8 * chunks;
  const int tiles = (full + kMidKT - 1) / kMidKT;
  const float* xrow[2];
  const float* arow[4];
#pragma unroll
  for (int q = 0; q < 2; ++q) xrow[q] = x + (size_t)min(r0 + 2 * w + q, m - 1) * k;
#pragma unroll
  for (int q = 0; q < 4; ++q) arow[q] = a + (size_t)min(j0 + 4 * w + q, rank - 1) * k;
  auto issue = [&](int t) {
    const int kb = t * kMidKT;  // kb <= full - 8 <= k - 8
    const uint32_t off = 4u * (uint32_t)min(4 * lane, k - 4 - kb);
    float(*slot)[kMidStride] = lds[t % kMidSlots];
#pragma unroll
    for (int q = 0; q < 2; ++q) dma16s(xrow[q] + kb, off, slot[2 * w + q]);
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16s(arow[q] + kb, off, slot[kMidRows + 4 * w + q]);
  };
  const int i = (lane >> 2) & 7;
  const int xr = 4 * (lane >> 5) + (lane & 3), jl = 4 * w + (lane & 3);
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < kMidSlots - 1; ++t)
    if (t < tiles) issue(t);
  for (int t = 0; t < tiles; ++t) {
    // this wave's loads of tile t are done once at most the newer tiles' remain
    if (t + kMidSlots - 2 < tiles)
      wait_vmcnt<(kMidSlots - 2) * kMidLoads>();
    else
      wait_vmcnt<0>();
    lds_barrier();  // every wave's tile t has landed and tile t-1 is summed
    if (t + kMidSlots - 1 < tiles) issue(t + kMidSlots - 1);  // the slot of tile t-1
    const float* xs = lds[t % kMidSlots][xr] + i;
    const float* as = lds[t % kMidSlots][kMidRows + jl] + i;
    const int cmax = min(kMidKT / 8, chunks - t * (kMidKT / 8));
    if (cmax == kMidKT / 8) {
#if DQ8_MID_PIPE
      // a full tile in batches of kMidBatch chunks, software-pipelined in three
      // stages: the LDS operands of batch bt+2 are read while the products of
      // batch bt+1 are formed and batch bt is added (one wave per SIMD: nothing
      // else hides an LDS read or an MFMA issued just before its use)
      constexpr int NB = kMidKT / 8 / kMidBatch;
      float xo[2][kMidBatch], ao[2][kMidBatch];
      f32x4 d[2][kMidBatch];
      auto operands = [&](float(&xv)[kMidBatch], float(&av)[kMidBatch], int c0) {
#pragma unroll
        for (int u = 0; u < kMidBatch; ++u) {
          xv[u] = xs[8 * (c0 + u)];
          av[u] = as[8 * (c0 + u)];
        }
      };
      auto products = [&](f32x4(&o)[kMidBatch], const float(&xv)[kMidBatch], const float(&av)[kMidBatch]) {
#pragma unroll
        for (int u = 0; u < kMidBatch; ++u) o[u] = __builtin_amdgcn_mfma_f32_4x4x1f32(xv[u], av[u], zero, 0, 0, 0);
      };
      operands(xo[0], ao[0], 0);
      if (NB > 1) operands(xo[1], ao[1], kMidBatch);
      products(d[0], xo[0], ao[0]);
#pragma unroll
      for (int bt = 0; bt < NB; ++bt) {
        if (bt + 2 < NB) operands(xo[bt & 1], ao[bt & 1], kMidBatch * (bt + 2));
        __builtin_amdgcn_sched_barrier(0);
        if (bt + 1 < NB) products(d[(bt + 1) & 1], xo[(bt + 1) & 1], ao[(bt + 1) & 1]);
#pragma unroll
        for (int u = 0; u < kMidBatch; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = acc[r] + d[bt & 1][u][r];
      }
#else
      // a full tile in batches of kMidBatch chunks: the products of the next
      // batch are formed while the current batch is added
      constexpr int NB = kMidKT / 8 / kMidBatch;
      f32x4 d[2][kMidBatch];
      auto products = [&](f32x4(&o)[kMidBatch], int c0) {
        float xo[kMidBatch], ao[kMidBatch];
#pragma unroll
        for (int u = 0; u < kMidBatch; ++u) {
          xo[u] = xs[8 * (c0 + u)];
          ao[u] = as[8 * (c0 + u)];
        }
#pragma unroll
        for (int u = 0; u < kMidBatch; ++u) o[u] = __builtin_amdgcn_mfma_f32_4x4x1f32(xo[u], ao[u], zero, 0, 0, 0);
      };
      products(d[0], 0);
#pragma unroll
      for (int bt = 0; bt < NB; ++bt) {
        if (bt + 1 < NB) products(d[(bt + 1) & 1], kMidBatch * (bt + 1));
#pragma unroll
        for (int u = 0; u < kMidBatch; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = acc[r] + d[bt & 1][u][r];
      }
#endif
    } else {
      for (int c = 0; c < cmax; ++c) {
        const f32x4 d = __builtin_amdgcn_mfma_f32_4x4x1f32(xs[8 * c], as[8 * c], zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = acc[r] + d[r];
      }
    }
  }
  const int j = j0 + jl;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float sum = -0.0f;
#pragma unroll
    for (int ii = 0; ii < 8; ++ii) sum = sum + __shfl(acc[r], (lane & 32) + 4 * ii + (lane & 3));
    const int row = r0 + 4 * (lane >> 5) + r;
    if (i == 0 && row < m && j < rank) {
      const float* xg = x + (size_t)row * k;
      const float* ag = a + (size_t)j * k;
      for (int e = full; e < k; ++e) sum = sum + xg[e] * ag[e];
      mid[(size_t)row * rank + j] = sum + 0.0f;
    }
  }
}
__global__ __launch_bounds__(256) void k_lora_mid_dma(const float* __restrict__ x, int m, int k,
                                                      const float* __restrict__ a, int rank, float* __restrict__ mid) {
  __shared__ __attribute__((aligned(16))) MidTile lds;
  lora_mid_tiled(x, m, k, a, rank, mid, (int)blockIdx.x, lds);
}
// The item of block b of a grouped middle-product launch: the last one whose
// first block is <= b (block_begin ascends).  Unrolled over the table of first
// blocks, so its loads go out together rather than one round trip per item.
__device__ __forceinline__ int find_mid(const MidBatch& bt, int b) {
  int it = 0;
#pragma unroll
  for (int i = 1; i < kMaxMids; ++i)
    if (i < bt.count && b >= bt.block_begin[i]) it = i;
  return it;
}
// Several tiled middle products in one launch.
__global__ __launch_bounds__(256) void k_lora_mid_dma_batch(MidBatch bt) {
  __shared__ __attribute__((aligned(16))) MidTile lds;
  const int b = (int)blockIdx.x;
  const MidItem I = bt.it[find_mid(bt, b)];
  lora_mid_tiled(I.x, I.m, I.k, I.a, I.rank, I.mid, b - I.block_begin, lds);
}

// k_lora_mid_small<R, J>: few rows (m <= 32).  A block holds R whole rows of x
// and J whole adapter rows in LDS, fetched by one round of direct global->LDS
// loads (1 KB each; the block's 4 waves issue every 4th, at most 39 each), so
// the memory latency is paid once; then the first R * J * 8 threads compute.  Lane l works on row r0 + (l/8)/J, adapter row j0 + (l/8)%J and lane
// sum i = l%8: the chunks are summed in order on the VALU (one rounded product
// and one rounded add each), then the 8 lane sums of a pair, in consecutive
// lanes, are added in order from -0.0, then the tail elements.  Loads past a
// row's end are clamped to its last 16 bytes and land in the row padding.
// Requires k % 4 == 0, 16-byte aligned x and a, and roundup(k, 256) <= KR.
constexpr int kSmallR = 4, kSmallJ = 2, kSmallKR = 6656;  // the one configuration in use
constexpr int kSmallRS = kSmallKR + 8;                     // row stride: the 8 rows of a step in distinct banks
template <int R, int J, int KR>
__device__ __forceinline__ void lora_mid_small(const float* __restrict__ x, int m, int k, const float* __restrict__ a,
                                               int rank, float* __restrict__ mid, int block, float* lds) {
  constexpr int NT = R * J * 8, NW = 4, RS = KR + 8;
  static_assert(NT % 64 == 0 && NT <= 256, "whole waves of one block");
  static_assert((R + J) * ((KR + 255) / 256) <= 48 * NW, "at most 48 loads in flight per wave");
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int jblocks = (rank + J - 1) / J;
  const int r0 = (block / jblocks) * R, j0 = (block % jblocks) * J;
  const int segs = (k + 255) >> 8;  // 1 KB pieces per row
  for (int t = w; t < (R + J) * segs; t += NW) {  // wave-uniform
    const int row = t / segs, seg = t - row * segs;
    const float* src = row < R ? x + (size_t)min(r0 + row, m - 1) * k : a + (size_t)min(j0 + row - R, rank - 1) * k;
    const uint32_t off = 4u * (uint32_t)min(4 * lane, k - 4 - 256 * seg);  // k % 4 == 0: k - 256*seg >= 4
    dma16s(src + 256 * seg, off, lds + row * RS + 256 * seg);
  }
  wait_vmcnt<0>();
  lds_barrier();
  if (tid >= NT) return;  // wave-uniform: NT is a multiple of 64
  const int pr = tid >> 3, i = tid & 7, r = pr / J, j = pr - r * J;
  // Both row bases as opaque LDS addresses: the compiler would otherwise fold
  // the constant R * RS * 4 (over 64 KB) into every read's offset and, since
  // the offset field stops at 64 KB, rebuild each read's address on the VALU.
  typedef __attribute__((address_space(3))) const float* lds_row;
  lds_row xs = (lds_row)(lds + r * RS);
  lds_row as = (lds_row)(lds + (R + j) * RS);
  // this lane's elements i, i + 8, ...: one address step per CU chunks, the
  // chunks within it as immediate offsets; all CU chunks' operands are read
  // before the first is summed, so one LDS latency per CU chunks is exposed
  // (the chain's adds hide the rest)
  constexpr int CU = 32;
  lds_row xp = xs + i, ap = as + i;
  asm volatile("" : "+v"(xp), "+v"(ap));
  const int chunks = k >> 3;
  float acc = 0.0f;
  int c = 0;
  for (; c + CU <= chunks; c += CU, xp += 8 * CU, ap += 8 * CU) {
    float xv[CU], av[CU];
#pragma unroll
    for (int u = 0; u < CU; ++u) {
      xv[u] = xp[8 * u];
      av[u] = ap[8 * u];
    }
#pragma unroll
    for (int u = 0; u < CU; ++u) acc = acc + xv[u] * av[u];
  }
  for (; c < chunks; ++c, xp += 8, ap += 8) acc = acc + xp[0] * ap[0];
  float sum = -0.0f;
#pragma unroll
  for (int ii = 0; ii < 8; ++ii) sum = sum + __shfl(acc, (lane & ~7) + ii);
  const int row = r0 + r, jr = j0 + j;
  if (i == 0 && row < m && jr < rank) {
    for (int e = 8 * chunks; e < k; ++e) sum = sum + xs[e] * as[e];
    mid[(size_t)row * rank + jr] = sum + 0.0f;
  }
}
__global__ __launch_bounds__(256) void k_lora_mid_small(const float* __restrict__ x, int m, int k,
                                                        const float* __restrict__ a, int rank, float* __restrict__ mid) {
  __shared__ __attribute__((aligned(16))) float lds[(kSmallR + kSmallJ) * kSmallRS];
  lora_mid_small<kSmallR, kSmallJ, kSmallKR>(x, m, k, a, rank, mid, (int)blockIdx.x, lds);
}
// Several middle products in one launch (block -> item by find_mid).
__global__ __launch_bounds__(256) void k_lora_mid_small_batch(MidBatch bt) {
  __shared__ __attribute__((aligned(16))) float lds[(kSmallR + kSmallJ) * kSmallRS];
  const int b = (int)blockIdx.x;
  const MidItem I = bt.it[find_mid(bt, b)];
  lora_mid_small<kSmallR, kSmallJ, kSmallKR>(I.x, I.m, I.k, I.a, I.rank, I.mid, b - I.block_begin, lds);
}

// dot_scores (tensor.rs:6-25, the x86-64 order) of a[0..len) and b[0..len)
// from plain memory: eight lane sums over the full chunks of 8, added in
// order from -0.0, then the tail elements one by one; no fused multiply-add.
__device__ __forceinline__ float dot_scores_rows(const float* a, const float* b, int len) {
  const int chunks = len >> 3;
  float lanes[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < chunks; ++c)
#pragma unroll
    for (int q = 0; q < 8; ++q) lanes[q] = lanes[q] + a[8 * c + q] * b[8 * c + q];
  float sum = -0.0f;
#pragma unroll
  for (int q = 0; q < 8; ++q) sum = sum + lanes[q];
  for (int t = 8 * chunks; t < len; ++t) sum = sum + a[t] * b[t];
  return sum;
}

// Weight element (n, t) of the repacked layout, dequantized as Data::row does
// for 8-bit Quantized data (weights.rs:47-78): (float)(int8)q * scale.
__device__ __forceinline__ float dequant(const FProj& P, int n, int t) {
  const int g = t >> 6, off = t & 63, h = off >> 5, part = (off >> 4) & 1;
  const int8_t q = (int8_t)P.wt[((size_t)((n >> 5) * P.g + g) * 2 + h) * kFragBytes + ((n & 31) + 32 * part) * 16 +
                                (off & 15)];
  return (float)q * P.wst[(size_t)g * P.np + n];
}

// The FP32 path of a projection, Projection::columns_tiled (tensor.rs:206-269),
// which the crate takes when the inputs are not finite (tensor.rs:197-201):
//   y = dot_scores(x_r, w_n) + (bias[n] or 0.0)     w_n dequantized (dequant)
//   y = y + scale * (dot_scores(mid_r, B_n) + 0.0)   with an adapter (Adapter::combine)
// stored through the epilogue.  The dot products run in dot_scores' order, so
// NaN and infinity propagate as in the crate.  A block computes 32 rows x 64
// columns; thread (tr, tc) owns rows 2tr, 2tr+1 and columns tc + 16j (j < 4)
// with eight lane sums each.  Per group of 64 inputs the block stages x and
// the dequantized weights in LDS (rows padded to 68 floats: the 16 columns a
// wave reads per step fall in distinct banks).
constexpr int kF32Rows = 32, kF32Cols = 64, kF32Pad = 68;
__global__ __launch_bounds__(256) void k_linear_fp32(FProj P) {
  __shared__ __attribute__((aligned(16))) float xs[kF32Rows][kF32Pad];
  __shared__ __attribute__((aligned(16))) float ws[kF32Cols][kF32Pad];
  if (P.when && *P.when == 0) return;  // the inputs were finite: the int8 kernels ran
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int col_tiles = (P.n + kF32Cols - 1) / kF32Cols;
  const int m0 = (int)(blockIdx.x / col_tiles) * kF32Rows, n0 = (int)(blockIdx.x % col_tiles) * kF32Cols;
  const int chunks = P.k >> 3;  // full chunks of 8 go to the lane sums
  float acc[2][4][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[i][j][q] = 0.0f;
  for (int g = 0; 8 * g < chunks; ++g) {
    const int nfull = min(8, chunks - 8 * g);  // uniform over the block
    __syncthreads();                           // the previous group's reads are done
    {
      // x: thread t stages row t/8, inputs 64g + 8(t%8) .. +8 (zero past m or k)
      const int r = tid >> 3, seg = tid & 7, row = m0 + r, kk = 64 * g + 8 * seg;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        xs[r][8 * seg + u] = (row < P.m && kk + u < P.k) ? P.x[(size_t)row * P.k + kk + u] : 0.0f;
    }
    {
      // w: thread t stages column t/4, 16 inputs from one fragment lane (the
      // repacked layout is zero past n and k, and n0 + 63 < np)
      const int c = tid >> 2, h = (tid >> 1) & 1, part = tid & 1, n = n0 + c;
      const uint4 raw = *reinterpret_cast<const uint4*>(
          P.wt + ((size_t)((n >> 5) * P.g + g) * 2 + h) * kFragBytes + ((n & 31) + 32 * part) * 16);
      const float sc = P.wst[(size_t)g * P.np + n];
      const uint32_t word[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int u = 0; u < 16; ++u) ws[c][32 * h + 16 * part + u] = (float)(int8_t)(word[u >> 2] >> (8 * (u & 3))) * sc;
    }
    __syncthreads();
    for (int cc = 0; cc < nfull; ++cc) {
      float xv[2][8], wv[4][8];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float4 a = *reinterpret_cast<const float4*>(&xs[2 * tr + i][8 * cc]);
        const float4 b = *reinterpret_cast<const float4*>(&xs[2 * tr + i][8 * cc + 4]);
        xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
        xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 a = *reinterpret_cast<const float4*>(&ws[tc + 16 * j][8 * cc]);
        const float4 b = *reinterpret_cast<const float4*>(&ws[tc + 16 * j][8 * cc + 4]);
        wv[j][0] = a.x; wv[j][1] = a.y; wv[j][2] = a.z; wv[j][3] = a.w;
        wv[j][4] = b.x; wv[j][5] = b.y; wv[j][6] = b.z; wv[j][7] = b.w;
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[i][j][q] = acc[i][j][q] + xv[i][q] * wv[j][q];
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = m0 + 2 * tr + i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tc + 16 * j;
      if (row >= P.m || n >= P.n) continue;
      float y = -0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) y = y + acc[i][j][q];
      for (int t = 8 * chunks; t < P.k; ++t) y = y + P.x[(size_t)row * P.k + t] * dequant(P, n, t);
      y = y + (P.bias ? P.bias[n] : 0.0f);
      if (P.lora) {
        const float delta =
            (P.rank > 0 ? dot_scores_rows(P.lmid + (size_t)row * P.rank, P.lb + (size_t)n * P.rank, P.rank) : -0.0f) +
            0.0f;
        const float scaled = P.lscale * delta;
        y = y + scaled;
      }
      float* dst = P.layout == 1 ? P.out + (size_t)n * P.m + row : P.out + (size_t)row * P.n + n;
      if (P.epilogue == 0 || P.layout == 1) *dst = y;
      else if (P.epilogue == 1) *dst = *dst + y;
      else *dst = silu(*dst) * y;
    }
  }
}

}  // namespace

static unsigned blocks_for(long n, int per) { return (unsigned)((n + per - 1) / per); }

__global__ void k_fill_u32(uint32_t* p, uint32_t v) { *p = v; }
__global__ void k_or_u32(uint32_t* dst, const uint32_t* src) {
  if (*src) atomicOr(dst, *src);
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t v, hipStream_t s) {
  k_fill_u32<<<1, 1, 0, s>>>(p, v);
  return hipGetLastError();
}

hipError_t launch_or_u32(uint32_t* dst, const uint32_t* src, hipStream_t s) {
  k_or_u32<<<1, 1, 0, s>>>(dst, src);
  return hipGetLastError();
}

hipError_t launch_linear_fp32(const FProj& p, hipStream_t s) {
  if (p.m == 0 || p.n == 0) return hipSuccess;
  const long blocks = (long)((p.m + kF32Rows - 1) / kF32Rows) * ((p.n + kF32Cols - 1) / kF32Cols);
  k_linear_fp32<<<(unsigned)blocks, 256, 0, s>>>(p);
  return hipGetLastError();
}

bool lora_mid_small_ok(const float* x, int m, int k, const float* a) {
  return k % 4 == 0 && ((size_t)x & 15) == 0 && ((size_t)a & 15) == 0 && m <= DQ8_MID_SMALL_M &&
         ((k + 255) & ~255) <= kSmallKR;
}
long lora_mid_small_blocks(int m, int rank) { return (long)((m + kSmallR - 1) / kSmallR) * ((rank + kSmallJ - 1) / kSmallJ); }

bool lora_mid_tiled_ok(const float* x, int k, const float* a) {
  return k % 4 == 0 && ((size_t)x & 15) == 0 && ((size_t)a & 15) == 0;
}
long lora_mid_tiled_blocks(int m, int rank) {
  return (long)((m + kMidRows - 1) / kMidRows) * ((rank + kMidJ - 1) / kMidJ);
}

hipError_t launch_lora_mid_batch(const MidBatch& b, long blocks, bool tiled, hipStream_t s) {
  if (b.count == 0 || blocks == 0) return hipSuccess;
  if (tiled)
    k_lora_mid_dma_batch<<<(unsigned)blocks, 256, 0, s>>>(b);
  else
    k_lora_mid_small_batch<<<(unsigned)blocks, 256, 0, s>>>(b);
  return hipGetLastError();
}

hipError_t launch_lora_mid(const float* x, int m, int k, const float* a, int rank, float* mid, hipStream_t s) {
  if (m == 0 || rank == 0) return hipSuccess;
  const bool dma = k % 4 == 0 && ((size_t)x & 15) == 0 && ((size_t)a & 15) == 0;
  const int kr = (k + 255) & ~255;
  if (dma && m <= DQ8_MID_SMALL_M && kr <= kSmallKR) {
    // 4 x rows and 2 adapter rows per block (6 rows in LDS: the fewest for a
    // wave of lane sums); measured 6.1 us at 24 x 2048 rank 16 against 8.4 for
    // 8 x 4 blocks and 8.2 for the tiled kernel, 14.3 against 20.8 at k = 6144
    k_lora_mid_small<<<(unsigned)lora_mid_small_blocks(m, rank), 256, 0, s>>>(x, m, k, a, rank, mid);
  } else if (dma) {
    const long blocks = (long)((m + kMidRows - 1) / kMidRows) * ((rank + kMidJ - 1) / kMidJ);
    k_lora_mid_dma<<<(unsigned)blocks, 256, 0, s>>>(x, m, k, a, rank, mid);
  } else {
    const long waves = (long)((m + 3) / 4) * ((rank + 7) / 8);
    k_lora_mid_rows<<<blocks_for(waves, 4), 256, 0, s>>>(x, m, k, a, rank, mid);
  }
  return hipGetLastError();
}


hipError_t launch_quantize_raw(const void* x, int dtype, int rows, int k, int8_t* q, int ldq, float* scales, int lds,
                               uint32_t* nonfinite, hipStream_t s) {
#if DQ8_QUANT_LOOP > 0
  if (dtype == kDtypeF32 && k % 256 == 0 && ((uintptr_t)x & 15) == 0 && ldq % 4 == 0 && ((uintptr_t)q & 3) == 0) {
    const long total = (long)rows * (k / 256);
    if (total == 0) return hipSuccess;
    // the waves' chunk indices run to total + (DQ8_QUANT_LOOP + 1) * W (W <= 4 * kQuantLoopBlocks) in int
    if (total < (1L << 31) - (DQ8_QUANT_LOOP + 1) * (long)DQ8_QUANT_LOOP_WPB * kQuantLoopBlocks) {
      const int blocks = (int)std::min<long>(kQuantLoopBlocks, (total + DQ8_QUANT_LOOP_WPB - 1) / DQ8_QUANT_LOOP_WPB);
      k_quantize_loop<DQ8_QUANT_LOOP><<<blocks, 64 * DQ8_QUANT_LOOP_WPB, 0, s>>>(static_cast<const float*>(x), k, (int)total, q, ldq,
                                                             scales, lds, nonfinite, Divider::of((uint32_t)(k / 256)));
      return hipGetLastError();
    }
  }
#endif
  constexpr int PER = DQ8_QUANT_PER;
  const long waves = (long)rows * (((k + 255) / 256 + PER - 1) / PER);
  if (waves == 0) return hipSuccess;
  if (waves >= (1L << 31) - 4) return hipErrorInvalidValue;
  const int blocks = blocks_for(waves, DQ8_QUANT_WPB);
  const Divider wdiv = Divider::of((uint32_t)(((k + 255) / 256 + PER - 1) / PER));
  if (dtype == kDtypeBF16)
    k_quantize<kDtypeBF16, PER><<<blocks, 64 * DQ8_QUANT_WPB, 0, s>>>(x, rows, k, q, ldq, scales, lds, nonfinite, wdiv);
  else if (dtype == kDtypeF16)
    k_quantize<kDtypeF16, PER><<<blocks, 64 * DQ8_QUANT_WPB, 0, s>>>(x, rows, k, q, ldq, scales, lds, nonfinite, wdiv);
  else
    k_quantize<kDtypeF32, PER><<<blocks, 64 * DQ8_QUANT_WPB, 0, s>>>(x, rows, k, q, ldq, scales, lds, nonfinite, wdiv);
  return hipGetLastError();
}

hipError_t launch_quantize(const float* x, int rows, int k, int8_t* q, int ldq, float* scales, int lds,
                           uint32_t* nonfinite, hipStream_t s) {
  return launch_quantize_raw(x, kDtypeF32, rows, k, q, ldq, scales, lds, nonfinite, s);
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

hipError_t launch_pad_scales(const float* xs, int rows, int g, float* dst, int ld, hipStream_t s) {
  const long n = (long)rows * ld;
  if (n == 0) return hipSuccess;
  k_pad_scales<<<blocks_for(n, 256), 256, 0, s>>>(xs, rows, g, dst, ld);
  return hipGetLastError();
}

hipError_t launch_pad_rows(const int8_t* q, int rows, int k, int8_t* dst, int ldq, hipStream_t s) {
  k_pad_rows<<<blocks_for((long)rows * ldq, 256), 256, 0, s>>>(q, rows, k, dst, ldq);
  return hipGetLastError();
}

// Skinny launch shape (tunable at build time): a short-K wave covers 16*CT
// columns, a long-K wave 16*CTL; DBS / DBL steps in flight in their rings
// (DBS2 / DBL2 in the 17-32 row kernel).
#ifndef DQ8_SKINNY_CT
#define DQ8_SKINNY_CT 2
#endif
#ifndef DQ8_SKINNY_CTL
#define DQ8_SKINNY_CTL 1
#endif
#ifndef DQ8_SKINNY_DBS
#define DQ8_SKINNY_DBS 4
#endif
#ifndef DQ8_SKINNY_DBL
#define DQ8_SKINNY_DBL 6
#endif
#ifndef DQ8_SKINNY_DBS2
#define DQ8_SKINNY_DBS2 3  // the short-K ring of the 17-32 row kernel
#endif
#ifndef DQ8_SKINNY_DBL2
#define DQ8_SKINNY_DBL2 6  // the long-K ring of the 17-32 row kernel
#endif
// Short K (G <= 32) runs one wave per strip; longer K interleaves a strip's
// groups over 4 waves.
#ifndef DQ8_SKINNY_SHORT_MAX_G
#define DQ8_SKINNY_SHORT_MAX_G 32
#endif
int skinny_segments(int g, bool few_strips) { return g <= DQ8_SKINNY_SHORT_MAX_G && !few_strips ? 1 : 4; }
int skinny_cols(int nseg) { return 16 * (nseg == 1 ? DQ8_SKINNY_CT : DQ8_SKINNY_CTL); }
int wide_block_rows() { return 32 * DQ8_WIDE_RT * DQ8_WIDE_WM; }
int wide_block_cols() { return 32 * DQ8_WIDE_CT * DQ8_WIDE_WN; }
bool wide_can_pair() { return wide_pair_shape(DQ8_WIDE_WN, DQ8_WIDE_RT, DQ8_WIDE_CT); }

hipError_t launch_linear(const Batch& b, int kind, bool dots, hipStream_t s) {
  if (b.total_waves == 0) return hipSuccess;
  const bool lora = !dots && b.any_lora;
  if (kind == 0) {
    // total_waves counts blocks for the wide kernel.  Blocks that share a CU
    // with few others wait on load latency between groups; a ring one group
    // deeper hides it.  That is the case for launches of at most three blocks
    // per CU (the 2048-row stack's 512- and 768-block launches: 2.4% off its
    // step; at two blocks per CU a ring of 4, see DQ8_WIDE_DEEP4_BLOCKS), and for
    // the trailing long-K blocks of a launch that mixes long and short K (a
    // layer's projection set over a few questions' rows: 22-28% faster for
    // 96-192 rows, 1-3% at 384).  Above three blocks per CU the deeper ring's
    // 46 KB of LDS costs occupancy (1% on a 2048-row prefill).
    constexpr int threads = 64 * DQ8_WIDE_WM * DQ8_WIDE_WN;
    bool has_long = false, has_short = false;
    for (int i = 0; i < b.count; ++i) (b.p[i].g > 32 ? has_long : has_short) = true;
    const bool deep = b.total_waves <= DQ8_WIDE_DEEP_BLOCKS ||
                      (has_long && has_short && b.total_waves <= DQ8_WIDE_DEEP_MIXED);
#if DQ8_WIDE_PERSIST > 0
    const int grid = std::min(b.total_waves, DQ8_WIDE_PERSIST * 256);
#else
    const int grid = b.total_waves;
#endif
#define DQ8_WIDE(SA, SB, X, D, L)                                                                \
  k_linear_wide<DQ8_WIDE_WM, DQ8_WIDE_WN, DQ8_WIDE_RT, DQ8_WIDE_CT, SA, SB, X, DQ8_WIDE_SWZ, D, L> \
      <<<grid, threads, 0, s>>>(b)
    constexpr int S0 = DQ8_WIDE_STAGES, S1 = DQ8_WIDE_STAGES + 1, X = DQ8_WIDE_XCH;
    bool pair_lora = false;
    for (int i = 0; i < b.count; ++i) pair_lora |= b.p[i].pair && (b.p[i].lora || b.p[i].lora2);
    if (pair_lora) {  // a SwiGLU pair with adapters
      k_linear_wide<DQ8_WIDE_WM, DQ8_WIDE_WN, DQ8_WIDE_RT, DQ8_WIDE_CT, 2, 3, 8, DQ8_WIDE_SWZ, false, true, true>
          <<<grid, threads, 0, s>>>(b);
      return hipGetLastError();
    }
    if (dots) DQ8_WIDE(S0, S0, X, true, false);
    else if (b.total_waves <= DQ8_WIDE_DEEP4_BLOCKS) lora ? DQ8_WIDE(4, 4, X, false, true) : DQ8_WIDE(4, 4, X, false, false);
#if DQ8_WIDE_SPLIT == 0
    else if (lora) deep ? DQ8_WIDE(S1, S1, X, false, true) : DQ8_WIDE(S0, S0, X, false, true);
    else deep ? DQ8_WIDE(S1, S1, X, false, false) : DQ8_WIDE(S0, S0, X, false, false);
#elif DQ8_WIDE_SPLIT == 1
    else if (lora) deep ? DQ8_WIDE(S1, S1, X, false, true) : DQ8_WIDE(2, 3, 8, false, true);
    else deep ? DQ8_WIDE(S1, S1, X, false, false) : DQ8_WIDE(2, 3, 8, false, false);
#else
    else if (lora) DQ8_WIDE(2, 3, 8, false, true);
    else DQ8_WIDE(2, 3, 8, false, false);
#endif
#undef DQ8_WIDE
    return hipGetLastError();
  }
  // total_waves counts blocks of 4 waves for the skinny kernel; kind 1: M <= 16, kind 2: M <= 32
  constexpr int CT = DQ8_SKINNY_CT, CL = DQ8_SKINNY_CTL;
#define DQ8_SKINNY(R, D, L)                                                                                  \
  k_linear_skinny<R, CT, CL, (R == 1 ? DQ8_SKINNY_DBS : DQ8_SKINNY_DBS2), (R == 1 ? DQ8_SKINNY_DBL : DQ8_SKINNY_DBL2), \
                  D, L><<<b.total_waves, 256, 0, s>>>(b)
  if (kind == 1) {
    if (dots) DQ8_SKINNY(1, true, false);
    else if (lora) DQ8_SKINNY(1, false, true);
    else DQ8_SKINNY(1, false, false);
  } else {
    if (dots) DQ8_SKINNY(2, true, false);
    else if (lora) DQ8_SKINNY(2, false, true);
    else DQ8_SKINNY(2, false, false);
  }
#undef DQ8_SKINNY
  return hipGetLastError();
}

}  // namespace dq8

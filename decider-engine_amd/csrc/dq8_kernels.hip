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

// Epilogue::store (tensor.rs:92-99) through write_columns (tensor.rs:272-288).
__device__ __forceinline__ void store_out(const Proj& P, int row, int col, float y) {
  if (P.layout == 1) {
    P.out[(size_t)col * P.m + row] = y;
    return;
  }
  float* dst = P.out + (size_t)row * P.n + col;
  if (P.epilogue == 0) *dst = y;
  else if (P.epilogue == 1) *dst = *dst + y;
  else *dst = silu(*dst) * y;
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
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
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

__global__ void k_repack_scales(const float* __restrict__ scales, int n, int g, int np, float* __restrict__ wst) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)g * np) return;
  const int gi = (int)(i / np), col = (int)(i % np);
  wst[i] = col < n ? scales[(size_t)col * g + gi] : 0.0f;
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
// Wide projection kernel (M > 32).  Each wave owns a 64 x 64 output tile:
// row tiles r0, r1 (32 rows each) x column tiles j0, j1.  Per group, for each
// column tile j the pair (r0, j), (r1, j) shares one conversion MFMA and one
// product MFMA: A lane l carries x scale of row m0 + l, B lane l carries the
// w scale of column n0 + 32j + l%32.
template <bool DOTS>
__global__ __launch_bounds__(256) void k_linear_wide(Batch b) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= b.total_waves) return;
  const Proj& P = b.p[find_proj(b, wave)];
  const int w = wave - P.wave_begin;
  const int mt = w / P.waves_n, nt = w - mt * P.waves_n;
  const int m0 = mt * 64, n0 = nt * 64;
  const int G = P.g;

  const int r_lo = min(m0 + (lane & 31), P.m - 1);
  const int r_hi = min(m0 + 32 + (lane & 31), P.m - 1);
  const int8_t* pa0 = P.q + (size_t)r_lo * P.ldq + 16 * (lane >> 5);
  const int8_t* pa1 = P.q + (size_t)r_hi * P.ldq + 16 * (lane >> 5);
  const uint8_t* pb0 = P.wt + (size_t)(n0 / 32) * G * 2 * kFragBytes + lane * 16;
  const uint8_t* pb1 = pb0 + (size_t)G * 2 * kFragBytes;
  const float* pxs = P.xs + (size_t)min(m0 + lane, P.m - 1) * G;
  const float* pws0 = P.wst + n0 + (lane & 31);
  const float* pws1 = pws0 + 32;

  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; ++i) magic[i] = kMagicBits;
  v32f zero32;
#pragma unroll
  for (int i = 0; i < 32; ++i) zero32[i] = 0.0f;
  v32f s0 = zero32, s1 = zero32;

  v4i a00 = load16(pa0), a01 = load16(pa0 + 32), a10 = load16(pa1), a11 = load16(pa1 + 32);
  v4i b00 = load16(pb0), b01 = load16(pb0 + kFragBytes), b10 = load16(pb1), b11 = load16(pb1 + kFragBytes);
  // The dots kernels read no scales (their xs may be a placeholder).
  float xv = DOTS ? 0.0f : pxs[0], wv0 = DOTS ? 0.0f : pws0[0], wv1 = DOTS ? 0.0f : pws1[0];

  for (int g = 0; g < G; ++g) {
    const v4i ca00 = a00, ca01 = a01, ca10 = a10, ca11 = a11;
    const v4i cb00 = b00, cb01 = b01, cb10 = b10, cb11 = b11;
    const float cx = xv, cw0 = wv0, cw1 = wv1;
    if (g + 1 < G) {
      const int ao = (g + 1) * kGroup;
      const size_t bo = (size_t)(g + 1) * 2 * kFragBytes;
      a00 = load16(pa0 + ao); a01 = load16(pa0 + ao + 32);
      a10 = load16(pa1 + ao); a11 = load16(pa1 + ao + 32);
      b00 = load16(pb0 + bo); b01 = load16(pb0 + bo + kFragBytes);
      b10 = load16(pb1 + bo); b11 = load16(pb1 + bo + kFragBytes);
      if constexpr (!DOTS) {
        xv = pxs[g + 1];
        wv0 = pws0[(size_t)(g + 1) * P.np];
        wv1 = pws1[(size_t)(g + 1) * P.np];
      }
    }
    v16i d00 = mfma_i8(ca00, cb00, magic);
    d00 = mfma_i8(ca01, cb01, d00);
    v16i d10 = mfma_i8(ca10, cb00, magic);
    d10 = mfma_i8(ca11, cb01, d10);
    v16i d01 = mfma_i8(ca00, cb10, magic);
    d01 = mfma_i8(ca01, cb11, d01);
    v16i d11 = mfma_i8(ca10, cb10, magic);
    d11 = mfma_i8(ca11, cb11, d11);
    if constexpr (DOTS) {
      // dots[(row * N + col) * G + g] = dot_g for the four 32x32 tiles
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const v16i& d = t == 0 ? d00 : t == 1 ? d10 : t == 2 ? d01 : d11;
        const int rt = t & 1, ct = t >> 1;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + 32 * rt + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const int col = n0 + 32 * ct + (lane & 31);
          if (row < P.m && col < P.n) P.dots[((size_t)row * P.n + col) * G + g] = d[v] - kMagicBits;
        }
      }
    } else {
      const v32f dv0 = mfma_k1(-kMagic, 1.0f, concat(d00, d10));
      const v32f pv0 = mfma_k1(cx, cw0, zero32);
      const v32f dv1 = mfma_k1(-kMagic, 1.0f, concat(d01, d11));
      const v32f pv1 = mfma_k1(cx, cw1, zero32);
      s0 = s0 + dv0 * pv0;
      s1 = s1 + dv1 * pv1;
    }
  }
  if constexpr (!DOTS) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v32f& s = j == 0 ? s0 : s1;
      const int col = n0 + 32 * j + (lane & 31);
      if (col >= P.n) continue;
      const float bias = P.bias ? P.bias[col] : 0.0f;
#pragma unroll
      for (int v = 0; v < 32; ++v) {
        const int vv = v & 15;
        const int row = m0 + 32 * (v >> 4) + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);
        if (row < P.m) store_out(P, row, col, s[v] + bias);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny projection kernel (M <= 32): weight-streaming.  Each wave owns all
// (padded) 32 rows x one 32-column tile and walks the groups two at a time;
// the K=1 MFMAs pair group g (block 0) with group g+1 (block 1), and the fp32
// sum adds group g's terms before group g+1's.
template <bool DOTS>
__global__ __launch_bounds__(256) void k_linear_skinny(Batch b) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= b.total_waves) return;
  const Proj& P = b.p[find_proj(b, wave)];
  const int nt = wave - P.wave_begin;
  const int n0 = nt * 32;
  const int G = P.g;
  const int half = lane >> 5;

  const int row = min(lane & 31, P.m - 1);
  const int8_t* pa = P.q + (size_t)row * P.ldq + 16 * half;
  const uint8_t* pb = P.wt + (size_t)nt * G * 2 * kFragBytes + lane * 16;
  const float* pxs = P.xs + (size_t)row * G;
  const float* pws = P.wst + n0 + (lane & 31);

  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; ++i) magic[i] = kMagicBits;
  v32f zero32;
#pragma unroll
  for (int i = 0; i < 32; ++i) zero32[i] = 0.0f;
  v16f s;
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = 0.0f;

  const v4i z4 = {0, 0, 0, 0};
  for (int g = 0; g < G; g += 2) {
    const bool two = g + 1 < G;
    const v4i a00 = load16(pa + g * kGroup), a01 = load16(pa + g * kGroup + 32);
    const v4i b00 = load16(pb + (size_t)g * 2 * kFragBytes), b01 = load16(pb + (size_t)(g * 2 + 1) * kFragBytes);
    v4i a10 = z4, a11 = z4, b10 = z4, b11 = z4;
    if (two) {
      a10 = load16(pa + (g + 1) * kGroup); a11 = load16(pa + (g + 1) * kGroup + 32);
      b10 = load16(pb + (size_t)(g + 1) * 2 * kFragBytes);
      b11 = load16(pb + (size_t)((g + 1) * 2 + 1) * kFragBytes);
    }
    const int gl = g + half;  // group carried by this lane's half of the K=1 operands
    const float xv = (!DOTS && gl < G) ? pxs[gl] : 0.0f;
    const float wv = (!DOTS && gl < G) ? pws[(size_t)gl * P.np] : 0.0f;

    v16i d0 = mfma_i8(a00, b00, magic);
    d0 = mfma_i8(a01, b01, d0);
    v16i d1 = mfma_i8(a10, b10, magic);
    d1 = mfma_i8(a11, b11, d1);
    if constexpr (DOTS) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t == 1 && !two) break;
        const v16i& d = t == 0 ? d0 : d1;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = 8 * (v >> 2) + 4 * half + (v & 3);
          const int col = n0 + (lane & 31);
          if (r < P.m && col < P.n) P.dots[((size_t)r * P.n + col) * G + g + t] = d[v] - kMagicBits;
        }
      }
    } else {
      const v32f dv = mfma_k1(-kMagic, 1.0f, concat(d0, d1));
      const v32f pv = mfma_k1(xv, wv, zero32);
      const v32f t = dv * pv;
      s = s + __builtin_shufflevector(t, t, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
      s = s + __builtin_shufflevector(t, t, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
    }
  }
  if constexpr (!DOTS) {
    const int col = n0 + (lane & 31);
    if (col < P.n) {
      const float bias = P.bias ? P.bias[col] : 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = 8 * (v >> 2) + 4 * half + (v & 3);
        if (r < P.m) store_out(P, r, col, s[v] + bias);
      }
    }
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
  k_repack_scales<<<blocks_for((long)w->g * w->np, 256), 256, 0, s>>>(scales, n, w->g, w->np, w->scales);
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

hipError_t launch_linear(const Batch& b, int kind, bool dots, hipStream_t s) {
  if (b.total_waves == 0) return hipSuccess;
  const unsigned blocks = blocks_for(b.total_waves, 4);
  if (kind == 0) {
    if (dots) k_linear_wide<true><<<blocks, 256, 0, s>>>(b);
    else k_linear_wide<false><<<blocks, 256, 0, s>>>(b);
  } else {
    if (dots) k_linear_skinny<true><<<blocks, 256, 0, s>>>(b);
    else k_linear_skinny<false><<<blocks, 256, 0, s>>>(b);
  }
  return hipGetLastError();
}

}  // namespace dq8

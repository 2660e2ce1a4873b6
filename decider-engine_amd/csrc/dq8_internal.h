// Internal types shared by the HIP kernels (dq8_kernels.hip) and the C ABI
// implementation (dq8_api.hip).  Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dq8 {

constexpr int kGroup = 64;        // reference group width (weights.rs:119, tensor.rs:329)
constexpr int kFragBytes = 1024;  // one MFMA operand fragment: 64 lanes x 16 bytes
constexpr int kMaxBatch = 16;     // projections per launch
constexpr int kMaxMids = 32;      // LoRA middle products per grouped launch
constexpr int kColPad = 256;      // weights are padded to a multiple of this many outputs
// Stored element types of raw weights (values of dq8_dtype).
constexpr int kDtypeF32 = 0, kDtypeBF16 = 1, kDtypeF16 = 2;

// Repacked weights, owned by a dq8_weights handle.
//   values: [Np/32][G][2][64 lanes][16 bytes]; fragment (nb, g, h) holds, at lane l,
//           output row nb*32 + l%32 and input bytes g*64 + 32h + 16*(l/32) .. +16
//           (zero beyond N or K).
//   scales: [G + 1][Np] fp32, group-major (zero beyond N; row G all zero).
struct Weights {
  int device;
  int n, k, g, np;
  uint8_t* values;
  float* scales;
};

// Division by a fixed d >= 1 for 0 <= n < 2^31 without a divide (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994,
// Thm 4.2): with l = ceil(log2 d) and mul = ceil(2^(31+l) / d) < 2^32,
// floor(n / d) = (n * mul) >> (31 + l), since 0 <= mul*d - 2^(31+l) < d <= 2^l.
struct Divider {
  uint32_t mul;
  int shift;
  static Divider of(uint32_t d) {
    int l = 0;
    while ((1ull << l) < d) ++l;
    return {(uint32_t)(((1ull << (31 + l)) + d - 1) / d), 31 + l};
  }
  __host__ __device__ int div(uint32_t n) const { return (int)(((uint64_t)n * mul) >> shift); }
};

// One projection of a launch.  q is [M][ldq] bytes with ldq % 16 == 0 and
// every byte up to G*64 of each row readable (zero past K).
struct Proj {
  const int8_t* q;
  const float* xs;    // [M][ldxs], ldxs >= G
  const uint8_t* wt;  // Weights::values
  const float* wst;   // Weights::scales
  const float* bias;  // [N] or null
  float* out;
  int32_t* dots;      // debug output [M][N][G] (dots kernels only)
  const float* lmid;  // LoRA middle product [M][rank] (read only when rank > 0)
  const float* lb;    // LoRA B [N][rank]
  int lora;           // the projection has an adapter
  int rank;
  float lscale;
  int m, ldq, ldxs, g, n, np;
  int epilogue;       // 0 write, 1 add, 2 swiglu
  int layout;         // 0 rows [M][N], 1 columns [N][M]
  int wave_begin;     // first block of this projection in the launch
  int waves_n;        // column strips (wide: one block tile wide; skinny long K: 16 columns wide;
                      // skinny short K: 16-column units, dealt to blocks `units` at a time)
  int units;          // skinny short K: at most this many 16-column units per block (2..8)
  int deal_q, deal_r; // skinny short K: the waves_n units over B = ceil(waves_n / units) blocks,
                      // deal_q = waves_n / B each and one more for the first deal_r = waves_n % B
  int xcd_gm;         // wide: row bands of the per-XCD tile regions (1, 2, 4, 8), 0 = row-major order
  int xcd_sr, xcd_sc; // wide: a region is walked in chunks of xcd_sr row tiles x xcd_sc column tiles
  // wide: the tile walk's divisors, set with the fields above: region size in
  // row and column tiles, log2 of the 8 / xcd_gm column bands, and dividers by
  // waves_n, xcd_sr * xcd_rn, xcd_sr * xcd_sc and xcd_sr
  int xcd_rm, xcd_rn, xcd_gn_shift;
  Divider d_cols, d_band, d_chunk, d_sr;
  int nseg;           // skinny: waves per strip (1 or 4)
  // Fused SwiGLU pair (wide kernel only): wt/wst/bias are the gate weights,
  // wt2/wst2/bias2 the up weights of the same shape; the launch stores
  // h = silu(gate(x) + bias) * (up(x) + bias2) into out [M][N].  With hq
  // set it also quantizes h as k_quantize does: hq [M][N] int8, hs [M][G_h]
  // scales (G_h = ceil(N / 64)), 1 ORed into *hflag if h is not finite.
  const uint8_t* wt2;
  const float* wst2;
  const float* bias2;
  int8_t* hq;
  float* hs;
  uint32_t* hflag;
  int pair;
  // The up projection's LoRA adapter in a pair launch (lmid/lb/rank/lscale of
  // the fields above are the gate's).
  const float* lmid2;
  const float* lb2;
  int lora2;
  int rank2;
  float lscale2;
};

struct Batch {
  Proj p[kMaxBatch];
  int wave_begin[kMaxBatch];  // p[i].wave_begin, contiguous: one scalar load finds a block's projection
  int count;
  int total_waves;  // blocks of the launch
  int any_lora;     // some projection has a LoRA adapter (selects the kernels with the LoRA epilogue)
  // When set, the launch does nothing if *unless != 0: the inputs were not
  // finite and the FP32 kernel (k_linear_fp32) computes these outputs instead.
  const uint32_t* unless;
};

// LoRA middle products of several (x, A) pairs in one launch of the few-rows
// kernel (lora_mid_small_ok items) or of the LDS-tiled kernel.
struct MidItem {
  const float* x;
  const float* a;
  float* mid;
  int m, k, rank;
  int block_begin;  // first block of the item in the launch
};
struct MidBatch {
  MidItem it[kMaxMids];
  int block_begin[kMaxMids];  // it[i].block_begin, contiguous: two scalar loads find a block's item
  int count;
};

// One projection of the FP32 path (Projection::columns_tiled, tensor.rs:206-269)
// over fp32 inputs x [m][k] and dequantized int8 weights.
struct FProj {
  const float* x;
  const uint8_t* wt;  // Weights::values
  const float* wst;   // Weights::scales
  const float* bias;  // [n] or null
  const float* lmid;  // LoRA middle product [m][rank] (rank > 0)
  const float* lb;    // LoRA B [n][rank]
  int lora, rank;
  float lscale;
  float* out;
  int m, k, g, n, np;
  int epilogue, layout;
  const uint32_t* when;  // if set, the launch does nothing unless *when != 0
};

// Kernel launchers (dq8_kernels.hip).  All return hipError_t of the launch.
// scales row stride lds >= G = ceil(k / 64)
hipError_t launch_quantize(const float* x, int rows, int k, int8_t* q, int ldq, float* scales, int lds,
                           uint32_t* nonfinite, hipStream_t s);
// The same over raw stored elements of type dtype (kDtype*), decoded exactly.
hipError_t launch_quantize_raw(const void* x, int dtype, int rows, int k, int8_t* q, int ldq, float* scales, int lds,
                               uint32_t* nonfinite, hipStream_t s);
hipError_t launch_repack(const uint8_t* values, const float* scales, int n, int k, Weights* w, hipStream_t s);
hipError_t launch_export(const Weights* w, uint8_t* values, float* scales, hipStream_t s);
hipError_t launch_pad_rows(const int8_t* q, int rows, int k, int8_t* dst, int ldq, hipStream_t s);
hipError_t launch_pad_scales(const float* xs, int rows, int g, float* dst, int ld, hipStream_t s);
// *p = v, as a kernel (graph-capturable, unlike a memset node).
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, hipStream_t s);
// *dst |= *src on the device.
hipError_t launch_or_u32(uint32_t* dst, const uint32_t* src, hipStream_t s);
// The FP32 path of a projection (see FProj).
hipError_t launch_linear_fp32(const FProj& p, hipStream_t s);
// LoRA middle product mid [m][rank] = dot_scores(x_r, a_j) + 0.0 (x [m][k], a [rank][k]).
hipError_t launch_lora_mid(const float* x, int m, int k, const float* a, int rank, float* mid, hipStream_t s);
bool lora_mid_small_ok(const float* x, int m, int k, const float* a);  // the few-rows kernel takes it
long lora_mid_small_blocks(int m, int rank);
bool lora_mid_tiled_ok(const float* x, int k, const float* a);  // otherwise the LDS-tiled kernel, if this holds
long lora_mid_tiled_blocks(int m, int rank);
hipError_t launch_lora_mid_batch(const MidBatch& b, long blocks, bool tiled, hipStream_t s);
// Kind: 0 wide (M > 32), 1 skinny (M <= 16), 2 skinny (16 < M <= 32).  dots
// selects the debug kernel.
constexpr int kKinds = 3;
hipError_t launch_linear(const Batch& b, int kind, bool dots, hipStream_t s);
// Columns of a skinny strip for g groups (all rows), and the waves that share
// a strip's groups (1 or 4).
// Skinny kernel paths: 1 segment (one wave per strip, all groups; short K) or
// 4 (a strip's groups split over 4 waves; long K, or launches with few strips).
int skinny_segments(int g, bool few_strips);
int skinny_cols(int nseg);  // strip width of a path
// Block tile of the wide kernel (rows, columns); kColPad is a multiple of the columns.
int wide_block_rows();
int wide_block_cols();
// Whether this build's wide-kernel tile shape has the SwiGLU pair mode (the
// kernel ignores Proj::pair otherwise).
bool wide_can_pair();

}  // namespace dq8

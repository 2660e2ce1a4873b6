// C ABI of include/dq8.h on top of the HIP kernels in dq8_kernels.hip.
#include "../../include/dq8.h"
#include "dq8_internal.h"
#include "dq8_st.h"

#include <algorithm>
#include <mutex>
#include <new>
#include <stdint.h>
#include <string.h>
#include <vector>

// Scratch of dq8_apply_noalloc: its non-finite flag (first 256 bytes), then
// the quantized inputs and their scales.  Each device holds its own copy for
// the life of the process; host code uses only the per-device address that
// hipGetSymbolAddress returns (dq8_create looks it up once per device).
constexpr size_t kScratchFlagBytes = 256;
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchFlagBytes + kScratchBytes];

struct dq8_ctx {
  int device;
  // Workspace for padded / freshly quantized activations.  Grows, never shrinks;
  // only dq8_linear_f32in and K % 64 != 0 inputs use it.
  void* work = nullptr;
  size_t work_bytes = 0;
  // Workspace of dq8_ffn (the re-quantized SwiGlu product and the down adapter's
  // middle product), kept apart from `work`, which the projections it launches use.
  void* chain = nullptr;
  size_t chain_bytes = 0;
  uint32_t* flag = nullptr;  // non-finite flag for synchronous checks
  // Two pinned host buffers through which weight loads stream to the device,
  // and the events of the copies out of them (created on first use).
  void* staging[2] = {nullptr, nullptr};
  hipEvent_t staged[2] = {nullptr, nullptr};
  // Device buffers of weight loads: the stored elements, and the quantized
  // values and scales before the repack.  Grow, never shrink.
  void* load_raw = nullptr;
  size_t load_raw_bytes = 0;
  void* load_tmp = nullptr;
  size_t load_tmp_bytes = 0;
  // Device buffers that were outgrown.  A graph captured earlier may still
  // reference them, so they are freed only by dq8_destroy.
  std::vector<void*> retired;
  // This device's address of `scratch` (null if the lookup failed).
  uint8_t* scratch = nullptr;
};

struct dq8_weights {
  dq8::Weights w;
};

namespace {

using dq8::kGroup;

size_t groups_of(size_t k) { return (k + kGroup - 1) / kGroup; }

struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// Per-device address of `scratch`, looked up once per device with that
// device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices] = {};

uint8_t* scratch_address(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[device]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess && p) g_scratch[device] = (uint8_t*)p;
  }
  return g_scratch[device];
}

dq8_status from_hip(hipError_t e) {
  if (e == hipSuccess) return DQ8_OK;
  if (e == hipErrorOutOfMemory) return DQ8_ERR_NOMEM;
  return DQ8_ERR_DEVICE;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Whether work on s would be recorded into a graph.  A failed query counts as
// capturing: HIP reports an error for the legacy NULL stream while another
// stream captures in global mode, and an allocation then would invalidate that
// capture.
bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone;
}

// While this thread allocates, another stream of the process may be capturing
// in global mode, where an allocation is an unsafe call that invalidates that
// capture (and HIP reports the NULL stream as not capturing meanwhile).  The
// library's own buffers belong to no graph, so the thread switches to relaxed
// mode around their allocation.
struct RelaxedCapture {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  bool swapped;
  RelaxedCapture() { swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess; }
  ~RelaxedCapture() {
    if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
  }
};

// Grow a context buffer to at least `bytes`.  Never while `s` is being
// captured (DQ8_ERR_CAPTURE: nothing is allocated or enqueued).  The old
// buffer is retired, not freed: work queued earlier, or a graph captured
// earlier, may still use it, so it lives until dq8_destroy.  Growth doubles,
// so the retired buffers together stay smaller than the current one.
dq8_status ensure_buffer(dq8_ctx* ctx, void*& buf, size_t& have, size_t bytes, hipStream_t s) {
  if (bytes <= have) return DQ8_OK;
  if (capturing(s)) return DQ8_ERR_CAPTURE;
  const size_t want = std::max(bytes, 2 * have);
  void* fresh = nullptr;
  RelaxedCapture relaxed;
  hipError_t e = hipMalloc(&fresh, want);
  if (e != hipSuccess) return from_hip(e);
  if (buf) {
    try {
      ctx->retired.push_back(buf);
    } catch (...) {
      (void)hipFree(fresh);
      return DQ8_ERR_NOMEM;
    }
  }
  buf = fresh;
  have = want;
  return DQ8_OK;
}
// Grow a weight-load staging buffer (load_raw, load_tmp).  Only the weight
// loads use these, and they synchronize before returning (and refuse a
// capturing stream), so no queued work or graph can hold the old buffer: it is
// freed at once and the new one is sized to the request.
dq8_status ensure_load_buffer(void*& buf, size_t& have, size_t bytes, hipStream_t s) {
  if (bytes <= have) return DQ8_OK;
  if (capturing(s)) return DQ8_ERR_CAPTURE;
  RelaxedCapture relaxed;
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return from_hip(e);
  if (buf) {
    (void)hipFree(buf);
    buf = nullptr;
    have = 0;
  }
  e = hipMalloc(&buf, bytes);
  if (e != hipSuccess) {
    buf = nullptr;
    return from_hip(e);
  }
  have = bytes;
  return DQ8_OK;
}
dq8_status ensure_work(dq8_ctx* ctx, size_t bytes, hipStream_t s) {
  return ensure_buffer(ctx, ctx->work, ctx->work_bytes, bytes, s);
}

// Weight shapes a handle can hold: n from 1 to 2^30 and k from 1 to 2^26 with
// n*k <= 2^40.  The bounds on k and on the w-scale table (G + 1 rows of np
// floats, the last row zero; under 4 GiB) let the projection kernels form each
// group's operand offsets in 32 bits (group offsets below 2^31).
bool weight_shape_ok(size_t n, size_t k) {
  if (n == 0 || k == 0 || n > (1u << 30) || k > (1u << 26) || n * k > ((size_t)1 << 40)) return false;
  const size_t np = (n + dq8::kColPad - 1) / dq8::kColPad * dq8::kColPad;
  return np * (groups_of(k) + 1) * sizeof(float) < ((size_t)1 << 32);
}

dq8_status make_weights(dq8_ctx* ctx, size_t n, size_t k, dq8_weights** out) {
  if (!weight_shape_ok(n, k)) return DQ8_ERR_SHAPE;
  dq8_weights* h = new (std::nothrow) dq8_weights();
  if (!h) return DQ8_ERR_NOMEM;
  h->w.device = ctx->device;
  h->w.n = (int)n;
  h->w.k = (int)k;
  h->w.g = (int)groups_of(k);
  h->w.np = (int)((n + dq8::kColPad - 1) / dq8::kColPad * dq8::kColPad);
  h->w.values = nullptr;
  h->w.scales = nullptr;
  hipError_t e = hipMalloc(&h->w.values, (size_t)h->w.np * h->w.g * kGroup);
  // One extra all-zero row of scales: the kernels read it for groups past the end.
  if (e == hipSuccess) e = hipMalloc(&h->w.scales, (size_t)h->w.np * (h->w.g + 1) * sizeof(float));
  if (e != hipSuccess) {
    (void)hipFree(h->w.values);
    (void)hipFree(h->w.scales);
    delete h;
    return from_hip(e);
  }
  *out = h;
  return DQ8_OK;
}

// Fill a launch item.  q must already satisfy the kernel's requirements.
void fill_proj(dq8::Proj& p, const dq8::Weights& w, const int8_t* q, int ldq, const float* xs, int ldxs, size_t m,
               const float* bias, float* out, int32_t* dots, int layout, int epilogue, const dq8_lora* lora) {
  p.lmid = lora ? lora->mid : nullptr;
  p.lb = lora ? lora->b : nullptr;
  p.lora = lora != nullptr;
  p.rank = lora ? (int)lora->rank : 0;
  p.lscale = lora ? lora->scale : 0.0f;
  p.q = q;
  p.xs = xs;
  p.ldxs = ldxs;
  p.wt = w.values;
  p.wst = w.scales;
  p.bias = bias;
  p.out = out;
  p.dots = dots;
  p.m = (int)m;
  p.ldq = ldq;
  p.g = w.g;
  p.n = w.n;
  p.np = w.np;
  p.epilogue = epilogue;
  p.layout = layout;
  p.wt2 = nullptr;
  p.wst2 = nullptr;
  p.bias2 = nullptr;
  p.hq = nullptr;
  p.hs = nullptr;
  p.hflag = nullptr;
  p.pair = 0;
  p.lmid2 = nullptr;
  p.lb2 = nullptr;
  p.lora2 = 0;
  p.rank2 = 0;
  p.lscale2 = 0.0f;
}

// Wide kernel: split the tile grid into gm x gn regions, gm * gn = 8, one per
// XCD.  An XCD then fetches 1/gm of the activation rows and 1/gn of the weight
// columns into its L2, so the launch fetches about gn*|A| + gm*|B| bytes from
// beyond L2; pick the split that minimises it.  0 = no split (tile counts that
// no split divides).
int xcd_rows_split(int row_tiles, int col_tiles, size_t a_bytes, size_t b_bytes) {
  int best = 0;
  size_t best_cost = 0;
  for (int gm = 1; gm <= 8; gm *= 2) {
    const int gn = 8 / gm;
    if (row_tiles % gm != 0 || col_tiles % gn != 0) continue;
    const size_t cost = (size_t)gn * a_bytes + (size_t)gm * b_bytes;
    if (best == 0 || cost < best_cost) {
      best = gm;
      best_cost = cost;
    }
  }
  return best;
}

// Blocks of one launch that an XCD runs at the same time (32 CUs x 4 blocks).
#ifndef DQ8_XCD_SLOTS
#define DQ8_XCD_SLOTS 128
#endif
// Walk order within an XCD's region (tile_of): bands of sr row tiles, each in
// chunks of sc column tiles.  A chunk of about DQ8_XCD_SLOTS tiles runs at
// once; pick the sr (a divisor of the region's row tiles) whose chunk touches
// the fewest operand bytes: sr row tiles of activations plus sc column tiles
// of weights (a column tile of a SwiGLU pair holds both projections' rows).
void xcd_chunks(dq8::Proj& p, int row_tiles) {
  p.xcd_sr = 1;
  p.xcd_sc = 1;
  if (p.xcd_gm == 0) return;
  const int rm = row_tiles / p.xcd_gm, rn = p.waves_n / (8 / p.xcd_gm);
  const double a_tile = (double)dq8::wide_block_rows(), b_tile = (double)dq8::wide_block_cols();
  double best = -1.0;
  for (int sr = 1; sr <= rm; ++sr) {
    if (rm % sr) continue;
    const int sc = std::min(rn, std::max(1, (DQ8_XCD_SLOTS + sr - 1) / sr));
    const double cost = (sr * a_tile + sc * b_tile) / ((double)sr * sc);  // operand rows per tile
    if (best < 0 || cost < best) {
      best = cost;
      p.xcd_sr = sr;
      p.xcd_sc = sc;
    }
  }
}

// Kernel kind of a projection (see launch_linear).
int kind_of(const dq8::Weights&, size_t m) { return m > 32 ? 0 : m > 16 ? 2 : 1; }

// A skinny launch whose projections would run on fewer 32-column strips than
// this takes the 4-wave path for all of them: each wave then streams a quarter
// of a strip's groups, so 4x the waves keep weight loads in flight.  Measured
// at 24 rows, graph-replayed, 4-wave path against short-K blocks of dealt
// units: 2048x2048 (64 strips) 4.9 against 8.0 us, o + GDN out (128) 7.6
// against 8.3 us, 2048x6144 (192) 10.6 against 8.3 us, GDN in (257) 10.4
// against 8.2 us.
constexpr long kSkinnyFewStrips = 160;
long short_strips(const dq8::Weights& w) { return (w.n + dq8::skinny_cols(1) - 1) / dq8::skinny_cols(1); }
// 16-column units of a short-K projection (one-wave strips hold two).
long short_units(const dq8::Weights& w) { return w.g <= 32 ? (w.n + 15) / 16 : 0; }
// Units per block of a skinny launch's short-K projections.  The units spread
// over about one block per CU, at most 7 per block, two (one strip) at least:
// each CU streams its bytes at a limited rate, so the CU holding the most
// bytes sets the launch's time (24 rows, graph-replayed: GDN in alone 10.4 ->
// 8.3 us, gate+up 11.0 -> 8.8 us against 8-unit blocks of 4 whole strips on
// fewer CUs).  Launches with long-K projections deal them the same way: the
// 24-row 9-projection layer set went 3.42 -> 3.51 TB/s per question
// (graph-replayed, 5 rotating weight copies).  (8 would select blocks of 4
// whole 32-column strips, one per wave.)
#ifndef DQ8_SKINNY_UNITS_MAX
#define DQ8_SKINNY_UNITS_MAX 7
#endif
int units_per_block(long units, bool /*has_long*/) {
  return (int)std::min((long)DQ8_SKINNY_UNITS_MAX, std::max(2L, (units + 255) / 256));
}

// Row chunks for the skinny kernel.  Up to 64 rows (rows layout) always run as
// chunks of at most 32 rows on the skinny kernel.  65-512 rows do when the
// call's wide launch would be small: at most kSplitWideBlocks blocks (under one
// block per CU, so every block would run alone on its CU and wait out each
// group's dependency chain), at most kSplitBytes of weights read by all the
// chunks (the first read comes from HBM, the rest mostly from cache), and no
// projection's weights above kSplitWeightBytes (larger ones are re-read from
// the MALL rather than L2).  Rows are independent, so the results are the same
// bits either way.  Measured (graph-replayed launches, wide -> chunks):
// 128 x 2048 -> 2048 17.5 -> 10.2 us, 128 x 2048 -> 6144 18.1 -> 10.9 us,
// 192 x 2048 -> 6144 18.4 -> 14.7 us, 192 x 6144 -> 2048 Add 48.1 -> 38.1 us,
// 512 x 2048 -> 2048 18.3 -> 12.6 us.  The chunks lost for 128 x 2048 -> 8224
// (18.7 -> 20.1 us), 256 x 6144 -> 2048 Add (48.3 -> 50.3 us) and 384 x 2048
// -> 6144 (23.6 -> 24.1 us).
constexpr long kSplitWideBlocks = 192;
constexpr double kSplitBytes = 96e6;
constexpr double kSplitWeightBytes = 16e6;
double weight_bytes(const dq8::Weights& w) { return (double)w.n * w.k + 4.0 * w.n * w.g; }
bool may_split(const dq8::Weights& w, size_t m, int layout) {
  return kind_of(w, m) == 0 && layout == DQ8_ROWS && (m <= 64 || (m <= 512 && weight_bytes(w) <= kSplitWeightBytes));
}
long wide_blocks(const dq8::Weights& w, size_t m) {
  return (long)((m + dq8::wide_block_rows() - 1) / dq8::wide_block_rows()) * (w.np / dq8::wide_block_cols());
}
size_t row_chunks(const dq8::Weights& w, size_t m, int layout, bool small_call) {
  if (!may_split(w, m, layout) || (m > 64 && !small_call)) return 1;
  return (m + 31) / 32;
}
// Whether a call's 65-512-row items run as skinny row chunks (see row_chunks).
template <class Item, class W>
bool small_call(const Item* items, size_t count, W weights_of) {
  long blocks = 0;
  double bytes = 0;
  for (size_t i = 0; i < count; ++i) {
    const dq8::Weights& w = weights_of(items[i]);
    const size_t m = items[i].m;
    if (m == 0 || kind_of(w, m) != 0) continue;
    const bool can = may_split(w, m, items[i].layout);
    if (can && m <= 64) continue;  // split whatever the call
    blocks += wide_blocks(w, m);
    if (can) bytes += (double)((m + 31) / 32) * weight_bytes(w);
  }
  return blocks <= kSplitWideBlocks && bytes <= kSplitBytes;
}

// Place a filled projection in a launch of the given kernel kind: its first
// wave/block, column strips, XCD split and the launch's running total.
void place_proj(dq8::Proj& p, int kind, dq8::Batch& b, bool few_strips, long launch_units, bool launch_has_long) {
  p.wave_begin = b.total_waves;
  b.wave_begin[&p - b.p] = p.wave_begin;
  p.xcd_gm = 0;
  p.nseg = 1;
  if (kind == 0) {
    // a SwiGLU pair's block covers half as many outputs of each projection
    p.waves_n = p.pair ? (p.n + dq8::wide_block_cols() / 2 - 1) / (dq8::wide_block_cols() / 2)
                       : p.np / dq8::wide_block_cols();
    const int row_tiles = (p.m + dq8::wide_block_rows() - 1) / dq8::wide_block_rows();
    p.xcd_gm = xcd_rows_split(row_tiles, p.waves_n, (size_t)p.m * p.g, (size_t)(p.pair ? 2 : 1) * p.n * p.g);
    xcd_chunks(p, row_tiles);
    p.d_cols = dq8::Divider::of((uint32_t)std::max(1, p.waves_n));
    if (p.xcd_gm) {
      const int gn = 8 / p.xcd_gm;
      p.xcd_rm = row_tiles / p.xcd_gm;
      p.xcd_rn = p.waves_n / gn;
      p.xcd_gn_shift = gn == 8 ? 3 : gn == 4 ? 2 : gn == 2 ? 1 : 0;
      p.d_band = dq8::Divider::of((uint32_t)(p.xcd_sr * p.xcd_rn));
      p.d_chunk = dq8::Divider::of((uint32_t)(p.xcd_sr * p.xcd_sc));
      p.d_sr = dq8::Divider::of((uint32_t)p.xcd_sr);
    }
    b.total_waves += p.waves_n * row_tiles;
  } else {
    p.nseg = dq8::skinny_segments(p.g, few_strips);
    if (p.nseg == 1) {
      // short K: 16-column units dealt to blocks, units_per_block at a time
      p.waves_n = (p.n + 15) / 16;
      p.units = units_per_block(launch_units, launch_has_long);
      const int blocks = (p.waves_n + p.units - 1) / p.units;
      p.deal_q = p.waves_n / blocks;
      p.deal_r = p.waves_n % blocks;
      b.total_waves += blocks;
    } else {
      // long K: one 16-row tile of a strip per block (kind 2: two per strip)
      p.waves_n = (p.n + dq8::skinny_cols(p.nseg) - 1) / dq8::skinny_cols(p.nseg);
      b.total_waves += p.waves_n * (kind == 2 ? 2 : 1);
    }
  }
}

// Quantized inputs are usable by the kernels directly when rows are 16-byte
// aligned and every group is complete; otherwise they are copied, zero-padded
// to G*64 bytes per row, into the context workspace.
bool needs_pad(const dq8::Weights& w, const int8_t* q) { return w.k % kGroup != 0 || !aligned(q, 16); }
size_t pad_bytes(const dq8::Weights& w, size_t m) { return (m * (size_t)w.g * kGroup + 255) / 256 * 256; }
// The kernels load x scales in 16-byte pieces of 4 groups: rows must be
// 16-byte aligned with a stride that is a multiple of 4 floats.  Otherwise they
// are copied into the workspace with the stride rounded up (zero past G).
int padded_groups(const dq8::Weights& w) { return (w.g + 3) / 4 * 4; }
bool needs_xs_pad(const dq8::Weights& w, const float* xs) { return w.g % 4 != 0 || !aligned(xs, 16); }
size_t xs_pad_bytes(const dq8::Weights& w, size_t m) {
  return (m * (size_t)padded_groups(w) * sizeof(float) + 255) / 256 * 256;
}

// A LoRA pair needs its two matrices unless its rank is 0 (then only the
// crate's `+ scale * (0.0 + 0.0)` remains); mid [m][rank] and b [n][rank] are
// read at rank floats per row.
dq8_status check_lora(const dq8_lora* lora) {
  if (!lora) return DQ8_OK;
  if (lora->rank > (1u << 20)) return DQ8_ERR_SHAPE;
  if (lora->rank > 0 && (!lora->mid || !lora->b)) return DQ8_ERR_ARG;
  return DQ8_OK;
}

dq8_status check_item_args(const dq8_weights* w, const int8_t* q, const float* scales, size_t m, float* out,
                           dq8_layout layout, dq8_epilogue epilogue) {
  if (!w || !q || !scales || !out) return DQ8_ERR_ARG;
  if (layout != DQ8_ROWS && layout != DQ8_COLUMNS) return DQ8_ERR_ARG;
  if (epilogue != DQ8_WRITE && epilogue != DQ8_ADD && epilogue != DQ8_SWIGLU) return DQ8_ERR_ARG;
  if (layout == DQ8_COLUMNS && epilogue != DQ8_WRITE) return DQ8_ERR_ARG;
  // at most 2^39 outputs per item: a launch's block count (at least 64 x 64
  // outputs per block, summed over the 16 items a batch holds) then stays
  // below 2^31
  if (m > (1u << 30) || m * w->w.n > ((size_t)1 << 39)) return DQ8_ERR_SHAPE;
  return DQ8_OK;
}

// Quantized copy of a projection's stored result: q [m][n], scales [m][G].
struct QOut {
  int8_t* q;
  float* scales;
  uint32_t* nonfinite;
};

// Split items by kernel kind and launch.  Items with m == 0 do nothing (tensor.rs:152-154).
// qout (one item only): the item's stored result is then quantized by k_quantize.
// (Only the SwiGLU pair launch, run_pair, quantizes its result in its own
// epilogue; the step's other quantized inputs come from outside the projections.)
// unless: the launches do nothing on the device if *unless != 0 (the inputs
// were not finite; the caller runs the FP32 kernel for these items).
dq8_status run_linear(dq8_ctx* ctx, const dq8_linear_item* items, size_t count, int32_t* dots, hipStream_t s,
                      const QOut* qout = nullptr, const uint32_t* unless = nullptr) {
  size_t need = 0;
  for (size_t i = 0; i < count; ++i) {
    if (!items[i].m) continue;
    if (needs_pad(items[i].w->w, items[i].q)) need += pad_bytes(items[i].w->w, items[i].m);
    if (!dots && needs_xs_pad(items[i].w->w, items[i].scales))
      need += xs_pad_bytes(items[i].w->w, items[i].m);
  }
  if (need) {
    dq8_status st = ensure_work(ctx, need, s);
    if (st != DQ8_OK) return st;
  }
  dq8::Batch batch[dq8::kKinds];
  for (dq8::Batch& b : batch) {
    b.count = b.total_waves = b.any_lora = 0;
    b.unless = unless;
  }
  const bool small = small_call(items, count, [](const dq8_linear_item& it) -> const dq8::Weights& { return it.w->w; });
  // one-wave strips each skinny launch would have (see kSkinnyFewStrips)
  long strips[dq8::kKinds] = {}, units[dq8::kKinds] = {};
  bool has_long[dq8::kKinds] = {};
  for (size_t i = 0; i < count; ++i) {
    const dq8_linear_item& it = items[i];
    if (it.m == 0) continue;
    const size_t nch = row_chunks(it.w->w, it.m, it.layout, small);
    const int kind = nch > 1 ? 2 : kind_of(it.w->w, it.m);
    strips[kind] += (long)nch * short_strips(it.w->w);
    units[kind] += (long)nch * short_units(it.w->w);
    has_long[kind] = has_long[kind] || it.w->w.g > 32;
  }
  size_t offset = 0;
  // Two passes: projections with long K (more than 32 groups) first, so their
  // blocks start when the launch does instead of trailing the short ones.
  for (int pass = 0; pass < 2; ++pass)
  for (size_t i = 0; i < count; ++i) {
    const dq8_linear_item& it = items[i];
    if (it.m == 0) continue;
    const dq8::Weights& w = it.w->w;
    if ((w.g > 32) != (pass == 0)) continue;
    const int8_t* q = it.q;
    int ldq = w.k;
    if (needs_pad(w, it.q)) {
      int8_t* dst = (int8_t*)ctx->work + offset;
      ldq = w.g * kGroup;
      hipError_t e = dq8::launch_pad_rows(it.q, (int)it.m, w.k, dst, ldq, s);
      if (e != hipSuccess) return from_hip(e);
      q = dst;
      offset += pad_bytes(w, it.m);
    }
    const float* xs = it.scales;
    int ldxs = w.g;
    if (!dots && needs_xs_pad(w, it.scales)) {  // the dots kernels read no scales
      float* dst = (float*)((char*)ctx->work + offset);
      ldxs = padded_groups(w);
      hipError_t e = dq8::launch_pad_scales(it.scales, (int)it.m, w.g, dst, ldxs, s);
      if (e != hipSuccess) return from_hip(e);
      xs = dst;
      offset += xs_pad_bytes(w, it.m);
    }
    // Row chunks of at most 32 rows on the skinny kernel (row_chunks): for 33-64
    // rows the weights are read twice (the chunks run side by side, so mostly
    // once from HBM), which beats a wide launch of half-empty row tiles whose
    // long-K blocks trail (measured 44 against 52 us for 48 rows of a layer's
    // projection set).  Rows are independent, so the results are the same bits.
    const size_t nch = row_chunks(w, it.m, it.layout, small);
    const int kind = nch > 1 ? 2 : kind_of(w, it.m);
    const size_t half = (it.m + nch - 1) / nch;
    for (size_t r0 = 0; r0 < it.m; r0 += half) {
      const size_t rows = std::min(half, it.m - r0);
      dq8::Batch& b = batch[kind];
      if (b.count == dq8::kMaxBatch) {
        hipError_t e = dq8::launch_linear(b, kind, dots != nullptr, s);
        if (e != hipSuccess) return from_hip(e);
        b.count = 0;
        b.total_waves = 0;
        b.any_lora = 0;
      }
      dq8::Proj& p = b.p[b.count++];
      // (the dots kernels read neither x scales nor out, which may be stand-ins)
      fill_proj(p, w, q + r0 * ldq, ldq, dots ? xs : xs + r0 * ldxs, ldxs, rows, it.bias,
                dots ? it.out : it.out + r0 * w.n, dots ? dots + r0 * w.n * w.g : nullptr, it.layout, it.epilogue,
                dots ? nullptr : it.lora);
      if (p.lora) {
        p.lmid += r0 * p.rank;
        b.any_lora = 1;
      }
      place_proj(p, kind, b, strips[kind] < kSkinnyFewStrips, units[kind], has_long[kind]);
    }
  }
  for (int kind = 0; kind < dq8::kKinds; ++kind) {
    if (batch[kind].count == 0) continue;
    hipError_t e = dq8::launch_linear(batch[kind], kind, dots != nullptr, s);
    if (e != hipSuccess) return from_hip(e);
  }
  if (qout && count == 1 && items[0].m > 0) {
    const dq8::Weights& w = items[0].w->w;
    hipError_t e = dq8::launch_quantize(items[0].out, (int)items[0].m, w.n, qout->q, w.n, qout->scales,
                                        (w.n + kGroup - 1) / kGroup, qout->nonfinite, s);
    if (e != hipSuccess) return from_hip(e);
  }
  return DQ8_OK;
}

// One layer's gate and up projections (same shape, shared quantized input)
// in one wide launch that stores h = silu(gate + bias + adapter) * (up + bias2
// + adapter2) into h [m][n] and, as qout asks, quantizes h in the same launch
// (q [m][n], scales [m][ceil(n/64)], the non-finite flag).  The results equal
// the separate Write and SwiGlu launches and k_quantize bit for bit: each
// output's arithmetic is unchanged, only the two tiles of one output sit in
// one wave, and a block holds whole 64-column groups of h.  gate_lora and
// up_lora are NULL or pass pair_lora_ok.
dq8_status run_pair(dq8_ctx* ctx, const dq8::Weights& g, const dq8::Weights& u, const int8_t* q, const float* xs,
                    size_t m, const float* gate_bias, const float* up_bias, const dq8_lora* gate_lora,
                    const dq8_lora* up_lora, float* h, const QOut* qout, hipStream_t s) {
  (void)ctx;
  dq8::Batch b;
  b.count = 1;
  b.total_waves = 0;
  b.any_lora = gate_lora != nullptr || up_lora != nullptr;
  b.unless = nullptr;
  dq8::Proj& p = b.p[0];
  fill_proj(p, g, q, g.k, xs, g.g, m, gate_bias, h, nullptr, DQ8_ROWS, DQ8_WRITE, gate_lora);
  p.wt2 = u.values;
  p.wst2 = u.scales;
  p.bias2 = up_bias;
  p.lmid2 = up_lora ? up_lora->mid : nullptr;
  p.lb2 = up_lora ? up_lora->b : nullptr;
  p.lora2 = up_lora != nullptr;
  p.rank2 = up_lora ? (int)up_lora->rank : 0;
  p.lscale2 = up_lora ? up_lora->scale : 0.0f;
  if (qout) {
    p.hq = qout->q;
    p.hs = qout->scales;
    p.hflag = qout->nonfinite;
  }
  p.pair = 1;
  place_proj(p, 0, b, false, 0, false);
  return from_hip(dq8::launch_linear(b, 0, false, s));
}

// ------------------------------------------------------- fp32-input paths

// Arguments of the entry points that take fp32 inputs x [m][k].
dq8_status check_f32in(const dq8_ctx* ctx, const dq8_weights* w, const float* x, size_t m, const float* out,
                       dq8_layout layout, dq8_epilogue epilogue, const dq8_lora* lora) {
  if (!ctx || !w) return DQ8_ERR_ARG;
  if (m == 0) return DQ8_OK;
  if (!x || !out) return DQ8_ERR_ARG;
  if (layout != DQ8_ROWS && layout != DQ8_COLUMNS) return DQ8_ERR_ARG;
  if (epilogue != DQ8_WRITE && epilogue != DQ8_ADD && epilogue != DQ8_SWIGLU) return DQ8_ERR_ARG;
  if (layout == DQ8_COLUMNS && epilogue != DQ8_WRITE) return DQ8_ERR_ARG;
  if (m > (1u << 30)) return DQ8_ERR_SHAPE;
  if (w->w.device != ctx->device) return DQ8_ERR_ARG;
  return check_lora(lora);
}

// Workspace of dq8_ffn for m rows of intermediate width inter and a down
// adapter of rank `rank`: q_h [m][inter], scales_h [m][G] (16-byte aligned),
// the down adapter's middle product [m][rank].
size_t chain_bytes(size_t m, size_t inter, size_t rank) {
  const size_t gh = (inter + kGroup - 1) / kGroup;
  return (m * inter + 255) / 256 * 256 + (m * gh * sizeof(float) + 255) / 256 * 256 + m * rank * sizeof(float);
}

// Inputs quantized into the context workspace: q with rows of G*64 bytes,
// scales with rows of a multiple of 4 groups.
struct WorkInputs {
  int8_t* q;
  int ldq;
  float* xs;
  int ldxs;
};

// Bytes of quantized inputs (rows of G*64 bytes) for m rows, and where the
// scales (rows of a multiple of 4 groups) start after them.
size_t work_q_bytes(const dq8::Weights& w, size_t m) { return (m * (size_t)w.g * kGroup + 255) / 256 * 256; }

// Inputs laid out at base: q, then the scales.
WorkInputs inputs_at(const dq8::Weights& w, size_t m, void* base) {
  WorkInputs in;
  in.q = (int8_t*)base;
  in.ldq = w.g * kGroup;
  in.xs = (float*)((char*)base + work_q_bytes(w, m));
  in.ldxs = padded_groups(w);
  return in;
}

// QuantizedInputs::new of x [m][w.k] into `in`.  *flag is cleared first (by a
// kernel, so the call can be graph-captured) and ends up non-zero if x holds
// a non-finite value.
dq8_status quantize_into(const dq8::Weights& w, const float* x, size_t m, const WorkInputs& in, uint32_t* flag,
                         hipStream_t s) {
  hipError_t e = dq8::launch_fill_u32(flag, 0, s);
  if (e == hipSuccess) e = dq8::launch_quantize(x, (int)m, w.k, in.q, in.ldq, in.xs, in.ldxs, flag, s);
  return from_hip(e);
}

// The same into the context workspace, with ctx->flag.
dq8_status quantize_to_work(dq8_ctx* ctx, const dq8::Weights& w, const float* x, size_t m, hipStream_t s,
                            WorkInputs& in) {
  dq8_status st = ensure_work(ctx, work_q_bytes(w, m) + xs_pad_bytes(w, m), s);
  if (st != DQ8_OK) return st;
  in = inputs_at(w, m, ctx->work);
  return quantize_into(w, x, m, in, ctx->flag, s);
}

// Waits for the stream and reports ctx->flag as DQ8_ERR_NONFINITE.
dq8_status finish_nonfinite(dq8_ctx* ctx, hipStream_t s) {
  uint32_t host = 0;
  hipError_t e = hipMemcpyAsync(&host, ctx->flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return from_hip(e);
  return host ? DQ8_ERR_NONFINITE : DQ8_OK;
}

// The int8 kernels for one projection over workspace inputs.
dq8_status launch_one(const dq8::Weights& w, const WorkInputs& in, size_t m, const float* bias, const dq8_lora* lora,
                      float* out, int layout, int epilogue, const uint32_t* unless, hipStream_t s) {
  dq8::Batch b;
  b.count = 1;
  b.total_waves = 0;
  b.any_lora = lora != nullptr;
  b.unless = unless;
  // (row chunks as in run_linear; at most 512 rows make at most 16 chunks)
  struct One {
    size_t m;
    int layout;
  } one = {m, layout};
  const size_t nch = row_chunks(w, m, layout, small_call(&one, 1, [&](const One&) -> const dq8::Weights& { return w; }));
  static_assert(dq8::kMaxBatch >= 16, "512 rows in chunks of 32");
  const int kind = nch > 1 ? 2 : kind_of(w, m);
  const size_t half = (m + nch - 1) / nch;
  b.count = 0;
  for (size_t r0 = 0; r0 < m; r0 += half) {
    dq8::Proj& p = b.p[b.count++];
    fill_proj(p, w, in.q + r0 * in.ldq, in.ldq, in.xs + r0 * in.ldxs, in.ldxs, std::min(half, m - r0), bias,
              out + r0 * w.n, nullptr, layout, epilogue, lora);
    if (p.lora) p.lmid += r0 * p.rank;
    place_proj(p, kind, b, (long)nch * short_strips(w) < kSkinnyFewStrips, (long)nch * short_units(w), w.g > 32);
  }
  return from_hip(dq8::launch_linear(b, kind, false, s));
}

// The FP32 path of a projection (k_linear_fp32) over x [m][w.k].
dq8::FProj make_fproj(const dq8::Weights& w, const float* x, size_t m, const float* bias, const dq8_lora* lora,
                      float* out, int layout, int epilogue, const uint32_t* when) {
  dq8::FProj p;
  p.x = x;
  p.wt = w.values;
  p.wst = w.scales;
  p.bias = bias;
  p.lora = lora != nullptr;
  p.rank = lora ? (int)lora->rank : 0;
  p.lscale = lora ? lora->scale : 0.0f;
  p.lmid = lora ? lora->mid : nullptr;
  p.lb = lora ? lora->b : nullptr;
  p.out = out;
  p.m = (int)m;
  p.k = w.k;
  p.g = w.g;
  p.n = w.n;
  p.np = w.np;
  p.epilogue = epilogue;
  p.layout = layout;
  p.when = when;
  return p;
}

// Projection::apply_quantized after the quantization of x into `in` with its
// non-finite flag: both paths are queued and the flag lets exactly one of them
// run on the device (tensor.rs:190-201), with no synchronization.
dq8_status apply_paths(const dq8::Weights& w, const float* x, size_t m, const float* bias, const dq8_lora* lora,
                       float* out, int layout, int epilogue, const WorkInputs& in, const uint32_t* flag,
                       hipStream_t s) {
  dq8_status st = launch_one(w, in, m, bias, lora, out, layout, epilogue, flag, s);
  if (st != DQ8_OK) return st;
  return from_hip(dq8::launch_linear_fp32(make_fproj(w, x, m, bias, lora, out, layout, epilogue, flag), s));
}

// ------------------------------------------------------------- weight loads

constexpr size_t kStagingBytes = 8u << 20;

// Copies `bytes` bytes of a host source to device memory dst through the
// context's two pinned staging buffers: fill(buffer, offset, count) writes
// source bytes [offset, offset + count) into a buffer (a memcpy or a file
// read) while the other buffer's copy is in flight.  On failure, copies
// already queued may still be running: the caller synchronizes `s` before dst
// is reused.
template <typename Fill>
dq8_status stage_to_device(dq8_ctx* ctx, uint8_t* dst, size_t bytes, hipStream_t s, Fill fill) {
  for (int b = 0; b < 2; ++b) {
    if (!ctx->staging[b]) {
      hipError_t e = hipHostMalloc(&ctx->staging[b], kStagingBytes, hipHostMallocDefault);
      if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->staged[b], hipEventDisableTiming);
      if (e != hipSuccess) return from_hip(e);
    } else if (hipEventSynchronize(ctx->staged[b]) != hipSuccess) {  // an earlier load's copy
      return DQ8_ERR_DEVICE;
    }
  }
  size_t i = 0;
  for (size_t off = 0; off < bytes; off += kStagingBytes, ++i) {
    const int b = (int)(i & 1);
    const size_t count = std::min(kStagingBytes, bytes - off);
    if (i >= 2 && hipEventSynchronize(ctx->staged[b]) != hipSuccess) return DQ8_ERR_DEVICE;
    if (!fill(ctx->staging[b], off, count)) return DQ8_ERR_IO;
    hipError_t e = hipMemcpyAsync(dst + off, ctx->staging[b], count, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipEventRecord(ctx->staged[b], s);
    if (e != hipSuccess) return from_hip(e);
  }
  return DQ8_OK;
}

size_t raw_element_bytes(int dtype) { return dtype == dq8::kDtypeF32 ? 4 : 2; }
bool raw_shape_ok(size_t n, size_t k) { return weight_shape_ok(n, k); }

// Data::quantize of n*k stored elements at device address raw (weights.rs:98-146),
// then the repack into a new handle.  Non-finite elements: DQ8_ERR_NONFINITE,
// as Data::read's "non-finite weights" (weights.rs:170-187).
dq8_status quantize_raw_weights(dq8_ctx* ctx, const void* raw, int dtype, size_t n, size_t k, hipStream_t s,
                                dq8_weights** out) {
  const size_t g = groups_of(k);
  const size_t vbytes = (n * k + 255) & ~(size_t)255;
  dq8_status st = ensure_load_buffer(ctx->load_tmp, ctx->load_tmp_bytes, vbytes + n * g * sizeof(float), s);
  if (st != DQ8_OK) return st;
  uint8_t* values = static_cast<uint8_t*>(ctx->load_tmp);
  float* scales = reinterpret_cast<float*>(values + vbytes);
  uint32_t flag = 0;
  hipError_t e = dq8::launch_fill_u32(ctx->flag, 0, s);
  if (e == hipSuccess)
    e = dq8::launch_quantize_raw(raw, dtype, (int)n, (int)k, (int8_t*)values, (int)k, scales, (int)g, ctx->flag, s);
  if (e == hipSuccess) e = hipMemcpyAsync(&flag, ctx->flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  st = from_hip(e);
  if (st == DQ8_OK && flag) st = DQ8_ERR_NONFINITE;
  if (st == DQ8_OK) st = dq8_weights_from_quantized(ctx, values, scales, n, k, s, out);
  (void)hipStreamSynchronize(s);  // the repack has read the buffers before another load reuses them
  return st;
}

// Stream n*k stored elements from a host source into a device buffer, then
// quantize and repack them.
template <typename Fill>
dq8_status load_weights(dq8_ctx* ctx, int dtype, size_t n, size_t k, hipStream_t s, dq8_weights** out, Fill fill) {
  const size_t bytes = n * k * raw_element_bytes(dtype);
  dq8_status st = ensure_load_buffer(ctx->load_raw, ctx->load_raw_bytes, bytes, s);
  if (st != DQ8_OK) return st;
  uint8_t* raw = static_cast<uint8_t*>(ctx->load_raw);
  st = stage_to_device(ctx, raw, bytes, s, fill);
  if (st == DQ8_OK) st = quantize_raw_weights(ctx, raw, dtype, n, k, s, out);
  (void)hipStreamSynchronize(s);
  return st;
}

bool dtype_ok(dq8_dtype d) { return d == DQ8_F32 || d == DQ8_BF16 || d == DQ8_F16; }

}  // namespace

extern "C" {

const char* dq8_status_string(dq8_status s) {
  switch (s) {
    case DQ8_OK: return "ok";
    case DQ8_ERR_SHAPE: return "shape mismatch";
    case DQ8_ERR_NONFINITE: return "non-finite input";
    case DQ8_ERR_ARG: return "invalid argument";
    case DQ8_ERR_DEVICE: return "device error";
    case DQ8_ERR_NOMEM: return "out of device memory";
    case DQ8_ERR_FORMAT: return "invalid safetensors data";
    case DQ8_ERR_IO: return "file read failed";
    case DQ8_ERR_CAPTURE: return "the call would allocate while its stream is being captured";
    case DQ8_ERR_LIMIT: return "the input exceeds the entry point's fixed scratch size";
  }
  return "unknown status";
}

dq8_status dq8_create(int device, dq8_ctx** out) {
  if (!out) return DQ8_ERR_ARG;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return DQ8_ERR_ARG;
  DeviceGuard guard(device);
  if (!guard.ok) return DQ8_ERR_DEVICE;
  dq8_ctx* ctx = new (std::nothrow) dq8_ctx();
  if (!ctx) return DQ8_ERR_NOMEM;
  ctx->device = device;
  hipError_t e = hipMalloc(&ctx->flag, sizeof(uint32_t));
  if (e != hipSuccess) {
    delete ctx;
    return from_hip(e);
  }
  ctx->scratch = scratch_address(device);  // null: dq8_apply_noalloc reports DQ8_ERR_DEVICE
  *out = ctx;
  return DQ8_OK;
}

dq8_status dq8_destroy(dq8_ctx* ctx) {
  if (!ctx) return DQ8_ERR_ARG;
  DeviceGuard guard(ctx->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(ctx->work);
  (void)hipFree(ctx->chain);
  (void)hipFree(ctx->flag);
  for (int b = 0; b < 2; ++b) {
    if (ctx->staged[b]) (void)hipEventDestroy(ctx->staged[b]);
    if (ctx->staging[b]) (void)hipHostFree(ctx->staging[b]);
  }
  (void)hipFree(ctx->load_raw);
  (void)hipFree(ctx->load_tmp);
  for (void* p : ctx->retired) (void)hipFree(p);
  delete ctx;
  return DQ8_OK;
}

dq8_status dq8_reserve(dq8_ctx* ctx, size_t m, size_t k, size_t rank) {
  if (!ctx) return DQ8_ERR_ARG;
  if (m > (1u << 30) || k > (1u << 30) || rank > (1u << 20) || m * k > ((size_t)1 << 40)) return DQ8_ERR_SHAPE;
  if (m == 0 || k == 0) return DQ8_OK;
  DeviceGuard guard(ctx->device);
  // the largest workspace of one projection with K <= k: quantized rows of
  // G*64 bytes plus scales rows of a multiple of 4 groups (dq8_apply,
  // dq8_linear_f32in), which also covers the padded copies of dq8_linear
  const size_t g = groups_of(k), gp = (g + 3) / 4 * 4;
  const size_t work = (m * g * kGroup + 255) / 256 * 256 + (m * gp * sizeof(float) + 255) / 256 * 256;
  dq8_status st = ensure_work(ctx, work, nullptr);
  if (st == DQ8_OK) st = ensure_buffer(ctx, ctx->chain, ctx->chain_bytes, chain_bytes(m, k, rank), nullptr);
  return st;
}

dq8_status dq8_weights_from_quantized(dq8_ctx* ctx, const uint8_t* values, const float* scales, size_t n, size_t k,
                                      void* stream, dq8_weights** out) {
  if (!ctx || !values || !scales || !out) return DQ8_ERR_ARG;
  *out = nullptr;
  DeviceGuard guard(ctx->device);
  dq8_weights* h = nullptr;
  dq8_status st = make_weights(ctx, n, k, &h);
  if (st != DQ8_OK) return st;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dq8::launch_repack(values, scales, (int)n, (int)k, &h->w, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    dq8_weights_free(h);
    return from_hip(e);
  }
  *out = h;
  return DQ8_OK;
}

dq8_status dq8_weights_from_f32(dq8_ctx* ctx, const float* w, size_t n, size_t k, void* stream, dq8_weights** out) {
  if (!ctx || !w || !out) return DQ8_ERR_ARG;
  *out = nullptr;
  if (!raw_shape_ok(n, k)) return DQ8_ERR_SHAPE;
  DeviceGuard guard(ctx->device);
  // Data::quantize has the same per-group formula as QuantizedInputs::new
  // (weights.rs:117-136); F32 elements decode to themselves, and non-finite
  // weights are rejected as the crate's loader rejects them (weights.rs:170-187).
  return quantize_raw_weights(ctx, w, dq8::kDtypeF32, n, k, (hipStream_t)stream, out);
}

dq8_status dq8_weights_from_raw(dq8_ctx* ctx, const void* data, dq8_dtype dtype, size_t n, size_t k, void* stream,
                                dq8_weights** out) {
  if (!ctx || !data || !out || !dtype_ok(dtype)) return DQ8_ERR_ARG;
  *out = nullptr;
  if (!raw_shape_ok(n, k)) return DQ8_ERR_SHAPE;
  DeviceGuard guard(ctx->device);
  return quantize_raw_weights(ctx, data, (int)dtype, n, k, (hipStream_t)stream, out);
}

dq8_status dq8_weights_upload(dq8_ctx* ctx, const void* data_host, dq8_dtype dtype, size_t n, size_t k,
                              void* stream, dq8_weights** out) {
  if (!ctx || !data_host || !out || !dtype_ok(dtype)) return DQ8_ERR_ARG;
  *out = nullptr;
  if (!raw_shape_ok(n, k)) return DQ8_ERR_SHAPE;
  DeviceGuard guard(ctx->device);
  const uint8_t* src = static_cast<const uint8_t*>(data_host);
  return load_weights(ctx, (int)dtype, n, k, (hipStream_t)stream, out, [&](void* buf, size_t off, size_t count) {
    memcpy(buf, src + off, count);
    return true;
  });
}

dq8_status dq8_st_load_weights(dq8_ctx* ctx, const dq8_st* st, size_t i, void* stream, dq8_weights** out) {
  if (!ctx || !st || !out || i >= st->tensors.size()) return DQ8_ERR_ARG;
  *out = nullptr;
  const dq8_st_tensor& t = st->tensors[i];
  const int dtype = dq8::st_dtype_code(t.dtype);
  if (dtype < 0) return DQ8_ERR_FORMAT;  // "unsupported weight dtype"
  // weights.rs:346-355: a 2-D projection weight with a non-zero width
  if (t.shape.size() != 2 || !raw_shape_ok(t.shape[0], t.shape[1])) return DQ8_ERR_SHAPE;
  DeviceGuard guard(ctx->device);
  const uint64_t base = st->data_start + t.begin;
  return load_weights(ctx, dtype, t.shape[0], t.shape[1], (hipStream_t)stream, out,
                      [&](void* buf, size_t off, size_t count) { return dq8::st_pread(st, buf, count, base + off); });
}

dq8_status dq8_weights_export(dq8_ctx* ctx, const dq8_weights* w, uint8_t* values, float* scales, void* stream) {
  if (!ctx || !w || !values || !scales) return DQ8_ERR_ARG;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dq8::launch_export(&w->w, values, scales, s);
  return from_hip(e);
}

dq8_status dq8_weights_shape(const dq8_weights* w, size_t* n, size_t* k) {
  if (!w || !n || !k) return DQ8_ERR_ARG;
  *n = (size_t)w->w.n;
  *k = (size_t)w->w.k;
  return DQ8_OK;
}

dq8_status dq8_weights_free(dq8_weights* w) {
  if (!w) return DQ8_ERR_ARG;
  DeviceGuard guard(w->w.device);
  (void)hipDeviceSynchronize();
  (void)hipFree(w->w.values);
  (void)hipFree(w->w.scales);
  delete w;
  return DQ8_OK;
}

dq8_status dq8_quantize(dq8_ctx* ctx, const float* x, size_t m, size_t k, int8_t* q, float* scales,
                        uint32_t* nonfinite, void* stream) {
  if (!ctx || (m && k && (!x || !q || !scales))) return DQ8_ERR_ARG;
  if (k == 0 || m > (1u << 30) || k > (1u << 30)) return DQ8_ERR_SHAPE;
  if (m == 0) return DQ8_OK;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  if (!nonfinite && capturing(s)) return DQ8_ERR_CAPTURE;  // it would synchronize
  uint32_t* flag = nonfinite ? nonfinite : ctx->flag;
  hipError_t e = hipSuccess;
  if (!nonfinite) e = dq8::launch_fill_u32(ctx->flag, 0, s);
  if (e == hipSuccess) e = dq8::launch_quantize(x, (int)m, (int)k, q, (int)k, scales, (int)groups_of(k), flag, s);
  if (e != hipSuccess) return from_hip(e);
  if (nonfinite) return DQ8_OK;
  uint32_t host = 0;
  e = hipMemcpyAsync(&host, ctx->flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return from_hip(e);
  return host ? DQ8_ERR_NONFINITE : DQ8_OK;
}

dq8_status dq8_linear(dq8_ctx* ctx, const dq8_weights* w, const int8_t* q, const float* scales, size_t m,
                      const float* bias, float* out, dq8_layout layout, dq8_epilogue epilogue, void* stream) {
  if (!ctx) return DQ8_ERR_ARG;
  if (m == 0) return w ? DQ8_OK : DQ8_ERR_ARG;
  dq8_status st = check_item_args(w, q, scales, m, out, layout, epilogue);
  if (st != DQ8_OK) return st;
  if (w->w.device != ctx->device) return DQ8_ERR_ARG;
  DeviceGuard guard(ctx->device);
  dq8_linear_item it = {w, q, scales, m, bias, out, layout, epilogue, nullptr};
  return run_linear(ctx, &it, 1, nullptr, (hipStream_t)stream);
}

dq8_status dq8_linear_lora(dq8_ctx* ctx, const dq8_weights* w, const int8_t* q, const float* scales, size_t m,
                           const float* bias, const dq8_lora* lora, float* out, dq8_layout layout,
                           dq8_epilogue epilogue, void* stream) {
  if (!ctx) return DQ8_ERR_ARG;
  if (m == 0) return w ? DQ8_OK : DQ8_ERR_ARG;
  dq8_status st = check_item_args(w, q, scales, m, out, layout, epilogue);
  if (st == DQ8_OK) st = check_lora(lora);
  if (st != DQ8_OK) return st;
  if (w->w.device != ctx->device) return DQ8_ERR_ARG;
  DeviceGuard guard(ctx->device);
  dq8_linear_item it = {w, q, scales, m, bias, out, layout, epilogue, lora};
  return run_linear(ctx, &it, 1, nullptr, (hipStream_t)stream);
}

}  // extern "C"

namespace {
// Arguments of one middle product (m == 0 or rank == 0: nothing to do).
dq8_status check_mid(const float* x, size_t m, size_t k, const float* a, size_t rank, const float* mid) {
  if (m == 0 || rank == 0) return DQ8_OK;
  if (!x || !a || !mid) return DQ8_ERR_ARG;
  if (k == 0 || m > (1u << 30) || k > (1u << 30) || rank > (1u << 20) || m * k > ((size_t)1 << 40) ||
      rank * k > ((size_t)1 << 40) || ((m + 7) / 8) * ((rank + 15) / 16) >= ((size_t)1 << 23))
    return DQ8_ERR_SHAPE;  // the last bound keeps the grid under 2^32 work-items
  return DQ8_OK;
}
// Whether the gate and up projections of an FFN can run as one SwiGLU pair
// launch: a wide-kernel build whose tile shape has the pair mode, the wide
// kernel (more than 64 rows), inputs the kernel reads as they are.
bool pair_ok(const dq8::Weights& g, const int8_t* q, const float* xs, size_t m) {
  return dq8::wide_can_pair() && kind_of(g, m) == 0 && m > 64 && !needs_pad(g, q) && !needs_xs_pad(g, xs);
}
// Adapters the pair launch's epilogue takes: rank 0, or rank 16 with 16-byte
// aligned mid and b (the rank of the reference's checkpoints); any other goes
// to the separate gate and up launches.
bool pair_lora_ok(const dq8_lora* l) {
  return !l || l->rank == 0 ||
         (l->rank == 16 && ((uintptr_t)l->mid & 15) == 0 && ((uintptr_t)l->b & 15) == 0);
}

// gate Write into h, then up SwiGlu into h; one launch when pair_ok.
dq8_status gate_up(dq8_ctx* ctx, const dq8_weights* gate, const dq8_weights* up, const int8_t* q, const float* xs,
                   size_t m, const float* gate_bias, const float* up_bias, const dq8_lora* gate_lora,
                   const dq8_lora* up_lora, float* h, const QOut* qout, hipStream_t s) {
  if (pair_ok(gate->w, q, xs, m) && pair_lora_ok(gate_lora) && pair_lora_ok(up_lora))
    return run_pair(ctx, gate->w, up->w, q, xs, m, gate_bias, up_bias, gate_lora, up_lora, h, qout, s);
  dq8_linear_item gi = {gate, q, xs, m, gate_bias, h, DQ8_ROWS, DQ8_WRITE, gate_lora};
  dq8_status st = run_linear(ctx, &gi, 1, nullptr, s);
  if (st != DQ8_OK) return st;
  dq8_linear_item ui = {up, q, xs, m, up_bias, h, DQ8_ROWS, DQ8_SWIGLU, up_lora};
  return run_linear(ctx, &ui, 1, nullptr, s, qout);
}

}  // namespace

extern "C" {

dq8_status dq8_lora_mid(dq8_ctx* ctx, const float* x, size_t m, size_t k, const float* a, size_t rank, float* mid,
                        void* stream) {
  if (!ctx) return DQ8_ERR_ARG;
  dq8_status st = check_mid(x, m, k, a, rank, mid);
  if (st != DQ8_OK || m == 0 || rank == 0) return st;
  DeviceGuard guard(ctx->device);
  return from_hip(dq8::launch_lora_mid(x, (int)m, (int)k, a, (int)rank, mid, (hipStream_t)stream));
}

dq8_status dq8_lora_mid_batch(dq8_ctx* ctx, const dq8_lora_mid_item* items, size_t count, void* stream) {
  if (!ctx || (count && !items)) return DQ8_ERR_ARG;
  for (size_t i = 0; i < count; ++i) {  // every item is checked before anything runs
    dq8_status st = check_mid(items[i].x, items[i].m, items[i].k, items[i].a, items[i].rank, items[i].mid);
    if (st != DQ8_OK) return st;
  }
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  // two grouped launches build up side by side: few-rows items and LDS-tiled items
  dq8::MidBatch b[2];
  long blocks[2] = {0, 0};
  b[0].count = b[1].count = 0;
  for (size_t i = 0; i < count; ++i) {
    const dq8_lora_mid_item& it = items[i];
    if (it.m == 0 || it.rank == 0) continue;
    const int m = (int)it.m, k = (int)it.k, rank = (int)it.rank;
    const bool small = dq8::lora_mid_small_ok(it.x, m, k, it.a);
    if (!small && !dq8::lora_mid_tiled_ok(it.x, k, it.a)) {  // the plain-memory kernel: a launch of its own
      hipError_t e = dq8::launch_lora_mid(it.x, m, k, it.a, rank, it.mid, s);
      if (e != hipSuccess) return from_hip(e);
      continue;
    }
    const int t = small ? 0 : 1;
    const long nb = small ? dq8::lora_mid_small_blocks(m, rank) : dq8::lora_mid_tiled_blocks(m, rank);
    if (b[t].count == dq8::kMaxMids || blocks[t] + nb >= ((long)1 << 23)) {
      hipError_t e = dq8::launch_lora_mid_batch(b[t], blocks[t], t == 1, s);
      if (e != hipSuccess) return from_hip(e);
      b[t].count = 0;
      blocks[t] = 0;
    }
    b[t].block_begin[b[t].count] = (int)blocks[t];
    b[t].it[b[t].count++] = {it.x, it.a, it.mid, m, k, rank, (int)blocks[t]};
    blocks[t] += nb;
  }
  for (int t = 0; t < 2; ++t) {
    hipError_t e = dq8::launch_lora_mid_batch(b[t], blocks[t], t == 1, s);
    if (e != hipSuccess) return from_hip(e);
  }
  return DQ8_OK;
}

dq8_status dq8_linear_batch(dq8_ctx* ctx, const dq8_linear_item* items, size_t count, void* stream) {
  if (!ctx || (count && !items)) return DQ8_ERR_ARG;
  for (size_t i = 0; i < count; ++i) {
    if (items[i].m == 0) {
      if (!items[i].w) return DQ8_ERR_ARG;
      continue;
    }
    dq8_status st = check_item_args(items[i].w, items[i].q, items[i].scales, items[i].m, items[i].out,
                                    items[i].layout, items[i].epilogue);
    if (st == DQ8_OK) st = check_lora(items[i].lora);
    if (st != DQ8_OK) return st;
    if (items[i].w->w.device != ctx->device) return DQ8_ERR_ARG;
  }
  DeviceGuard guard(ctx->device);
  return run_linear(ctx, items, count, nullptr, (hipStream_t)stream);
}

dq8_status dq8_ffn_gate_up_lora(dq8_ctx* ctx, const dq8_weights* gate, const dq8_weights* up, const int8_t* q,
                                const float* scales, size_t m, const float* gate_bias, const float* up_bias,
                                const dq8_lora* gate_lora, const dq8_lora* up_lora, float* h, int8_t* h_q,
                                float* h_scales, uint32_t* nonfinite, void* stream) {
  if (!ctx || !gate || !up) return DQ8_ERR_ARG;
  if (m == 0) return DQ8_OK;
  if (gate->w.k != up->w.k || gate->w.n != up->w.n) return DQ8_ERR_SHAPE;
  dq8_status st = check_item_args(gate, q, scales, m, h, DQ8_ROWS, DQ8_WRITE);
  if (st == DQ8_OK) st = check_lora(gate_lora);
  if (st == DQ8_OK) st = check_lora(up_lora);
  if (st != DQ8_OK) return st;
  if (gate->w.device != ctx->device || up->w.device != ctx->device) return DQ8_ERR_ARG;
  if ((h_q == nullptr) != (h_scales == nullptr)) return DQ8_ERR_ARG;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  if (!h_q) return gate_up(ctx, gate, up, q, scales, m, gate_bias, up_bias, gate_lora, up_lora, h, nullptr, s);
  if (!nonfinite && capturing(s)) return DQ8_ERR_CAPTURE;  // it would synchronize
  if (!nonfinite) {
    hipError_t e = dq8::launch_fill_u32(ctx->flag, 0, s);
    if (e != hipSuccess) return from_hip(e);
  }
  QOut qo = {h_q, h_scales, nonfinite ? nonfinite : ctx->flag};
  st = gate_up(ctx, gate, up, q, scales, m, gate_bias, up_bias, gate_lora, up_lora, h, &qo, s);
  if (st != DQ8_OK || nonfinite) return st;
  return finish_nonfinite(ctx, s);
}

dq8_status dq8_ffn_gate_up(dq8_ctx* ctx, const dq8_weights* gate, const dq8_weights* up, const int8_t* q,
                           const float* scales, size_t m, const float* gate_bias, const float* up_bias, float* h,
                           int8_t* h_q, float* h_scales, uint32_t* nonfinite, void* stream) {
  return dq8_ffn_gate_up_lora(ctx, gate, up, q, scales, m, gate_bias, up_bias, nullptr, nullptr, h, h_q, h_scales,
                              nonfinite, stream);
}

dq8_status dq8_linear_f32in(dq8_ctx* ctx, const dq8_weights* w, const float* x, size_t m, const float* bias,
                            float* out, dq8_layout layout, dq8_epilogue epilogue, void* stream) {
  dq8_status st = check_f32in(ctx, w, x, m, out, layout, epilogue, nullptr);
  if (st != DQ8_OK || m == 0) return st;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  if (capturing(s)) return DQ8_ERR_CAPTURE;  // it synchronizes
  WorkInputs in;
  st = quantize_to_work(ctx, w->w, x, m, s, in);
  if (st != DQ8_OK) return st;
  st = finish_nonfinite(ctx, s);
  if (st != DQ8_OK) return st;
  return launch_one(w->w, in, m, bias, nullptr, out, layout, epilogue, nullptr, s);
}

dq8_status dq8_linear_fp32(dq8_ctx* ctx, const dq8_weights* w, const float* x, size_t m, const float* bias,
                           const dq8_lora* lora, float* out, dq8_layout layout, dq8_epilogue epilogue, void* stream) {
  dq8_status st = check_f32in(ctx, w, x, m, out, layout, epilogue, lora);
  if (st != DQ8_OK || m == 0) return st;
  DeviceGuard guard(ctx->device);
  return from_hip(
      dq8::launch_linear_fp32(make_fproj(w->w, x, m, bias, lora, out, layout, epilogue, nullptr), (hipStream_t)stream));
}

dq8_status dq8_apply(dq8_ctx* ctx, const dq8_weights* w, const float* x, size_t m, const float* bias,
                     const dq8_lora* lora, float* out, dq8_layout layout, dq8_epilogue epilogue, void* stream) {
  dq8_status st = check_f32in(ctx, w, x, m, out, layout, epilogue, lora);
  if (st != DQ8_OK || m == 0) return st;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  WorkInputs in;
  st = quantize_to_work(ctx, w->w, x, m, s, in);
  if (st != DQ8_OK) return st;
  return apply_paths(w->w, x, m, bias, lora, out, layout, epilogue, in, ctx->flag, s);
}

dq8_status dq8_apply_noalloc(dq8_ctx* ctx, const dq8_weights* w, const float* x, size_t m, const float* bias,
                             const dq8_lora* lora, float* out, dq8_layout layout, dq8_epilogue epilogue,
                             void* stream) {
  dq8_status st = check_f32in(ctx, w, x, m, out, layout, epilogue, lora);
  if (st != DQ8_OK || m == 0) return st;
  if (work_q_bytes(w->w, m) + xs_pad_bytes(w->w, m) > kScratchBytes) return DQ8_ERR_LIMIT;
  if (!ctx->scratch) return DQ8_ERR_DEVICE;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  uint32_t* flag = reinterpret_cast<uint32_t*>(ctx->scratch);
  const WorkInputs in = inputs_at(w->w, m, ctx->scratch + kScratchFlagBytes);
  st = quantize_into(w->w, x, m, in, flag, s);
  if (st != DQ8_OK) return st;
  return apply_paths(w->w, x, m, bias, lora, out, layout, epilogue, in, flag, s);
}

dq8_status dq8_linear_q(dq8_ctx* ctx, const dq8_weights* w, const int8_t* q, const float* scales, size_t m,
                        const float* bias, const dq8_lora* lora, float* out, dq8_epilogue epilogue, int8_t* q_out,
                        float* scales_out, uint32_t* nonfinite, void* stream) {
  if (!ctx) return DQ8_ERR_ARG;
  if (m == 0) return w ? DQ8_OK : DQ8_ERR_ARG;
  dq8_status st = check_item_args(w, q, scales, m, out, DQ8_ROWS, epilogue);
  if (st == DQ8_OK) st = check_lora(lora);
  if (st != DQ8_OK) return st;
  if (!q_out || !scales_out) return DQ8_ERR_ARG;
  if (w->w.device != ctx->device) return DQ8_ERR_ARG;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  if (!nonfinite && capturing(s)) return DQ8_ERR_CAPTURE;  // it would synchronize
  if (!nonfinite) {
    hipError_t e = dq8::launch_fill_u32(ctx->flag, 0, s);
    if (e != hipSuccess) return from_hip(e);
  }
  QOut qo = {q_out, scales_out, nonfinite ? nonfinite : ctx->flag};
  dq8_linear_item it = {w, q, scales, m, bias, out, DQ8_ROWS, epilogue, lora};
  st = run_linear(ctx, &it, 1, nullptr, s, &qo);
  if (st != DQ8_OK || nonfinite) return st;
  return finish_nonfinite(ctx, s);
}

dq8_status dq8_ffn(dq8_ctx* ctx, const dq8_ffn_weights* f, const int8_t* q, const float* scales, size_t m, float* h,
                   float* residual, uint32_t* nonfinite, void* stream) {
  if (!ctx || !f || !f->gate || !f->up || !f->down) return DQ8_ERR_ARG;
  if (m == 0) return DQ8_OK;
  const dq8::Weights &g = f->gate->w, &u = f->up->w, &d = f->down->w;
  if (g.k != u.k || g.n != u.n || d.k != u.n) return DQ8_ERR_SHAPE;
  if (!q || !scales || !h || !residual) return DQ8_ERR_ARG;
  if (g.device != ctx->device || u.device != ctx->device || d.device != ctx->device) return DQ8_ERR_ARG;
  dq8_status st = check_lora(f->gate_lora);
  if (st == DQ8_OK) st = check_lora(f->up_lora);
  if (st != DQ8_OK) return st;
  const size_t rank = f->down_lora_a ? f->down_lora_rank : 0;
  if (f->down_lora_a && (!f->down_lora_b || rank == 0 || rank > (1u << 20))) return DQ8_ERR_ARG;
  if (m > (1u << 30) || m * std::max((size_t)u.n, (size_t)d.n) > ((size_t)1 << 39)) return DQ8_ERR_SHAPE;
  DeviceGuard guard(ctx->device);
  hipStream_t s = (hipStream_t)stream;
  // chain workspace: q_h [m][inter], scales_h [m][G] (16-byte aligned), down mid [m][rank]
  const size_t inter = (size_t)u.n, gh = (inter + kGroup - 1) / kGroup;
  const size_t qbytes = (m * inter + 255) / 256 * 256, sbytes = (m * gh * sizeof(float) + 255) / 256 * 256;
  (void)gh;
  st = ensure_buffer(ctx, ctx->chain, ctx->chain_bytes, chain_bytes(m, inter, rank), s);
  if (st != DQ8_OK) return st;
  int8_t* qh = (int8_t*)ctx->chain;
  float* sh = (float*)((char*)ctx->chain + qbytes);
  float* mid = (float*)((char*)ctx->chain + qbytes + sbytes);
  hipError_t e = dq8::launch_fill_u32(ctx->flag, 0, s);
  if (e != hipSuccess) return from_hip(e);
  // gate: Write into h (qwen.rs:489); up: SwiGlu into h (qwen.rs:490); h is
  // then quantized for down (qwen.rs:491).  Without adapters, on the wide
  // kernel, both projections run in one launch that stores h directly.
  QOut qo = {qh, sh, ctx->flag};
  st = gate_up(ctx, f->gate, f->up, q, scales, m, f->gate_bias, f->up_bias, f->gate_lora, f->up_lora, h, &qo, s);
  if (st != DQ8_OK) return st;
  if (nonfinite) {
    e = dq8::launch_or_u32(nonfinite, ctx->flag, s);
    if (e != hipSuccess) return from_hip(e);
  }
  // down: Add into the residual (qwen.rs:492), its adapter's middle product from h.
  // If h holds a non-finite value, QuantizedInputs::new(h) is None and the crate
  // takes the FP32 path on h (tensor.rs:197-201): both are queued and the flag
  // lets exactly one of them run on the device.
  dq8_lora dl = {mid, f->down_lora_b, rank, f->down_lora_scale};
  if (rank > 0) {
    e = dq8::launch_lora_mid(h, (int)m, (int)inter, f->down_lora_a, (int)rank, mid, s);
    if (e != hipSuccess) return from_hip(e);
  }
  const dq8_lora* dlp = f->down_lora_a ? &dl : nullptr;
  dq8_linear_item di = {f->down, qh, sh, m, f->down_bias, residual, DQ8_ROWS, DQ8_ADD, dlp};
  st = run_linear(ctx, &di, 1, nullptr, s, nullptr, ctx->flag);
  if (st != DQ8_OK) return st;
  return from_hip(
      dq8::launch_linear_fp32(make_fproj(d, h, m, f->down_bias, dlp, residual, DQ8_ROWS, DQ8_ADD, ctx->flag), s));
}

dq8_status dq8_group_dots(dq8_ctx* ctx, const dq8_weights* w, const int8_t* q, size_t m, int32_t* dots,
                          void* stream) {
  if (!ctx || !w || !q || !dots) return DQ8_ERR_ARG;
  if (m == 0) return DQ8_OK;
  DeviceGuard guard(ctx->device);
  // Scales are not read by the dots kernels; pass the weights' own as a valid pointer.
  dq8_linear_item it = {w, q, w->w.scales, m, nullptr, nullptr, DQ8_ROWS, DQ8_WRITE, nullptr};
  return run_linear(ctx, &it, 1, dots, (hipStream_t)stream);
}

}  // extern "C"

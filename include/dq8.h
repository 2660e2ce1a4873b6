/*
 * dq8.h -- C ABI of the MI355X (gfx950) INT8 linear-projection library.
 *
 * It is a drop-in for decider-engine's `int8-compute` projection path
 * (Rust crate decider-engine 0.2.2): group-64 symmetric int8 weights, per-token
 * group-64 activation quantization, exact i8*i8->i32 group dots and the
 * group-ordered fp32 rescale-and-sum.  Results are bit-identical to the
 * crate's CPU path.
 *
 * Conventions
 *   - Every pointer argument is a DEVICE pointer unless named *_host.
 *   - Callers own activations and outputs; the library owns repacked weights
 *     (dq8_weights) until dq8_weights_free, and its context workspace.
 *   - Nothing crosses the ABI as an exception: every entry returns dq8_status.
 *     Shape errors return DQ8_ERR_SHAPE where the crate panics (assert_eq!).
 *     A projection call also returns it for m > 2^30 rows or more than 2^39
 *     outputs (m * n) in one item, which keeps every launch's grid in range.
 *     Weight handles take n from 1 to 2^30 and k from 1 to 2^26 with
 *     n * k <= 2^40 and a scale table of ceil(n/256)*256 x (ceil(k/64) + 1)
 *     floats under 4 GiB (about 64 GiB of int8 weights); larger shapes return
 *     it too.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).
 *     Weight handles are immutable after creation, so calls on different
 *     streams may share them.  One context must not be used by two host
 *     threads at once, and its calls must be stream-ordered: the context's
 *     workspace and non-finite flag are single device buffers, so two calls of
 *     one context that use them (dq8_apply, dq8_linear_f32in, dq8_ffn,
 *     dq8_linear_q, dq8_quantize with nonfinite == NULL, and any projection
 *     whose q is not 16-byte aligned, whose k % 64 != 0 or whose scales rows
 *     are not 16-byte aligned with ceil(k/64) % 4 == 0) must not run
 *     concurrently on different streams.  Use one context per stream for
 *     concurrent work.
 *   - Graph capture: a call never allocates, frees or synchronizes while its
 *     stream is being captured.  If it would have to grow the context
 *     workspace it returns DQ8_ERR_CAPTURE and enqueues nothing; size the
 *     workspace first with dq8_reserve (or run the call once eagerly at the
 *     largest size).  A workspace that is outgrown is kept, not freed, until
 *     dq8_destroy, so graphs captured earlier stay valid.  Calls that
 *     synchronize by design (weight creation and loads, dq8_quantize /
 *     dq8_linear_q / dq8_ffn_gate_up with h_q, each with nonfinite == NULL,
 *     and dq8_linear_f32in) cannot be captured: on a capturing stream they
 *     return DQ8_ERR_CAPTURE and enqueue nothing.
 *   - The library starts no threads.
 *   - Weight loads keep their device buffers (stored elements, and values and
 *     scales before the repack) in the context, grown to the largest tensor
 *     loaded so far and freed by dq8_destroy.
 *
 * Layouts (M tokens, K input width, N outputs, G = ceil(K/64)):
 *   activations x  fp32 [M][K] row-major        (tensor.rs:315)
 *   quantized q    int8 [M][K], scales [M][G]   (QuantizedInputs, tensor.rs:310-313)
 *   weights        u8   [N][K], scales [N][G]   (Data::Quantized, weights.rs:16-23)
 *   result         fp32 [M][N] row-major        (write_columns, tensor.rs:272-288)
 *   columns        fp32 [N][M]                  (linear_int8's return, tensor.rs:441-455)
 */
#ifndef DQ8_H
#define DQ8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum dq8_status {
    DQ8_OK = 0,
    DQ8_ERR_SHAPE = 1,     /* a size or length disagrees (the crate's assert_eq! panics) */
    DQ8_ERR_NONFINITE = 2, /* QuantizedInputs::new returned None: caller takes its FP32 path */
    DQ8_ERR_ARG = 3,       /* null handle/pointer, bad enum value or misaligned pointer */
    DQ8_ERR_DEVICE = 4,    /* a HIP call failed */
    DQ8_ERR_NOMEM = 5,     /* device allocation failed */
    DQ8_ERR_FORMAT = 6,    /* a safetensors file or tensor that read_tensors / Data::read rejects */
    DQ8_ERR_IO = 7,        /* a file could not be opened or read */
    DQ8_ERR_CAPTURE = 8,   /* the stream is being captured and the call would allocate (see dq8_reserve) */
    DQ8_ERR_LIMIT = 9      /* the input exceeds the fixed scratch of dq8_apply_noalloc */
} dq8_status;

/* Stored element types of weights (Data::{F32, Bf16, F16}, weights.rs:12-15),
 * little-endian as in safetensors files. */
typedef enum dq8_dtype { DQ8_F32 = 0, DQ8_BF16 = 1, DQ8_F16 = 2 } dq8_dtype;

/* Epilogue::{Write, Add, SwiGlu} (tensor.rs:85-100). */
typedef enum dq8_epilogue { DQ8_WRITE = 0, DQ8_ADD = 1, DQ8_SWIGLU = 2 } dq8_epilogue;

/* Result layout: row-major [M][N] as written by write_columns (tensor.rs:272-288),
 * or the column-major [N][M] `columns` that linear_int8 returns (tensor.rs:441-455). */
typedef enum dq8_layout { DQ8_ROWS = 0, DQ8_COLUMNS = 1 } dq8_layout;

typedef struct dq8_ctx dq8_ctx;
typedef struct dq8_weights dq8_weights;

/* Context on one device.  Replaces the crate's implicit global state
 * (Kernel::detect, int8.rs:25-30, and the rayon pool). */
dq8_status dq8_create(int device, dq8_ctx **out);
dq8_status dq8_destroy(dq8_ctx *ctx);
/* Grow the context workspace, if needed, for calls of up to m rows of width
 * k: dq8_apply / dq8_linear_f32in / a padded dq8_linear of one projection with
 * K <= k, and dq8_ffn with an intermediate width <= k and a down adapter of
 * rank <= rank.  A dq8_linear_batch whose items need padding needs the sum of
 * their sizes.  Not capturable (it may allocate); no counterpart in the crate,
 * whose Vec buffers are allocated per call. */
dq8_status dq8_reserve(dq8_ctx *ctx, size_t m, size_t k, size_t rank);

/* Data::quantize(width, Precision::Int8Compute) (weights.rs:98-146) on the device,
 * from fp32 weights w [n][k], followed by the one-time repack into the
 * MFMA fragment layout.  A non-finite element returns DQ8_ERR_NONFINITE and
 * no handle, as the crate's loader rejects such weights before quantizing
 * them (Data::read, weights.rs:170-187).  Synchronous with respect to
 * `stream` on return of the handle (the handle is usable by later work on any
 * stream once `stream` has progressed past this call; dq8_weights_* calls
 * synchronize `stream`). */
dq8_status dq8_weights_from_f32(dq8_ctx *ctx, const float *w, size_t n, size_t k, void *stream,
                                dq8_weights **out);

/* Adopt an existing Data::Quantized { values, scales, width: k, bits: 8 }
 * (weights.rs:16-23) unchanged: values u8 [n][k] (i8 bit patterns),
 * scales fp32 [n][ceil(k/64)].  The crate's loader keeps quantizing on the
 * host; only the repack runs here. */
dq8_status dq8_weights_from_quantized(dq8_ctx *ctx, const uint8_t *values, const float *scales, size_t n,
                                      size_t k, void *stream, dq8_weights **out);

/* Data::read + Data::quantize(width, Precision::Int8Compute) of one projection
 * weight (weights.rs:147-195, 98-146, 346-355) from its stored elements: data
 * holds n*k elements of `dtype` in device memory.  Any non-finite element
 * returns DQ8_ERR_NONFINITE and no handle ("non-finite weights").  Elements are
 * decoded exactly (BF16: the upper half of an f32; F16: the IEEE conversion of
 * `half`, weights.rs:367-382), quantized in groups of 64 and repacked on the
 * device.  Synchronizes `stream`. */
dq8_status dq8_weights_from_raw(dq8_ctx *ctx, const void *data, dq8_dtype dtype, size_t n, size_t k, void *stream,
                                dq8_weights **out);
/* dq8_weights_from_raw with the elements in host memory (a read buffer or a
 * file mapping): they are streamed to the device through the context's two
 * pinned staging buffers, each refilled while the other one's copy runs. */
dq8_status dq8_weights_upload(dq8_ctx *ctx, const void *data_host, dq8_dtype dtype, size_t n, size_t k,
                              void *stream, dq8_weights **out);

/* Write the handle's weights back in the Data::Quantized layout (for checks). */
dq8_status dq8_weights_export(dq8_ctx *ctx, const dq8_weights *w, uint8_t *values, float *scales,
                              void *stream);
dq8_status dq8_weights_shape(const dq8_weights *w, size_t *n, size_t *k);
dq8_status dq8_weights_free(dq8_weights *w);

/* QuantizedInputs::new (tensor.rs:315-353): per token row, per group of 64,
 * symmetric absmax int8 and one fp32 scale.  If any element of x is
 * non-finite the crate returns None (tensor.rs:318-320):
 *   - nonfinite == NULL: the call synchronizes `stream` and returns
 *     DQ8_ERR_NONFINITE in that case (q/scales contents are then unspecified);
 *   - nonfinite != NULL: nothing is synchronized; the kernel ORs 1 into
 *     *nonfinite (a device uint32 the caller has zeroed) and returns DQ8_OK. */
dq8_status dq8_quantize(dq8_ctx *ctx, const float *x, size_t m, size_t k, int8_t *q, float *scales,
                        uint32_t *nonfinite, void *stream);

/* linear_int8 (tensor.rs:379-456) on quantized inputs q [m][k] / scales [m][G]
 * (a shared QuantizedInputs, tensor.rs:398-402), written through
 * write_columns + Epilogue (tensor.rs:272-288).  bias may be NULL (the crate adds
 * +0.0, tensor.rs:437).  For DQ8_COLUMNS the epilogue must be DQ8_WRITE. */
dq8_status dq8_linear(dq8_ctx *ctx, const dq8_weights *w, const int8_t *q, const float *scales, size_t m,
                      const float *bias, float *out, dq8_layout layout, dq8_epilogue epilogue, void *stream);

/* `linear` (tensor.rs:290-308) + epilogue: quantize x [m][k] and multiply.
 * Returns DQ8_ERR_NONFINITE (after synchronizing `stream`), leaving `out`
 * untouched, where the crate falls back to FP32 (tensor.rs:197-201). */
dq8_status dq8_linear_f32in(dq8_ctx *ctx, const dq8_weights *w, const float *x, size_t m, const float *bias,
                            float *out, dq8_layout layout, dq8_epilogue epilogue, void *stream);

/* The LoRA pair of a projection as Adapter (tensor.rs:102-108) holds it:
 *   mid   fp32 [m][rank]  the middle product x . A^T (dq8_lora_mid)
 *   b     fp32 [n][rank]  lora_B (weights.rs:427), the crate's FP32 Data::F32
 *   scale                 the adapter scale
 * Every output becomes y = (s + bias) + scale * (dot_scores(mid[row], b[col]) + 0.0)
 * (Adapter::combine, tensor.rs:109-117), with dot_scores in its x86-64 order
 * (tensor.rs:6-25) and every product and sum rounded on its own.  That is what
 * both of the crate's schedules produce: the per-output combine (m < 64) and the
 * separate B pass of Projection::apply_quantized (m >= 64, tensor.rs:155-179), and
 * the x86 plan of Linear::apply_into_shared (weights.rs:450-491).  The struct is
 * host memory; mid and b are device pointers. */
typedef struct dq8_lora {
    const float *mid;
    const float *b;
    size_t rank;
    float scale;
} dq8_lora;
/* LoRA middle product (Linear::apply_into_shared, weights.rs:480 and 495):
 * mid [m][rank] = linear(x, A) with x fp32 [m][k] and A = lora_A fp32 [rank][k],
 * i.e. mid[r][j] = dot_scores(x_r, A_j) + 0.0 (the FP32 columns of
 * tensor.rs:206-269 without bias).  Non-finite inputs propagate as in the crate.
 * DQ8_ERR_SHAPE for k == 0, m > 2^30, k > 2^30, rank > 2^20, m*k or rank*k
 * above 2^40, or ceil(m/8) * ceil(rank/16) >= 2^23. */
dq8_status dq8_lora_mid(dq8_ctx *ctx, const float *x, size_t m, size_t k, const float *a, size_t rank, float *mid,
                        void *stream);
/* Several middle products (dq8_lora_mid of each item) in as few launches as
 * possible: the projections of a question that carry adapters, each with its
 * own input x [m][k], lora_A [rank][k] and output mid [m][rank].  Items with
 * k % 4 == 0 and 16-byte aligned x and a share grouped launches of up to 32
 * items (one for items of at most 32 rows and k <= 6656, one for the others);
 * the rest run one launch each.  Every item is
 * checked as dq8_lora_mid checks it before anything is enqueued; the results
 * are those of dq8_lora_mid, bit for bit.  Items run concurrently: no item's
 * mid may overlap another item's x, a or mid.  No reference counterpart: the crate
 * computes each adapter's middle product in its own Linear::apply_into_shared
 * call (weights.rs:480, 495); this only schedules those products together. */
typedef struct {
    const float *x;
    size_t m, k;
    const float *a;
    size_t rank;
    float *mid;
} dq8_lora_mid_item;
dq8_status dq8_lora_mid_batch(dq8_ctx *ctx, const dq8_lora_mid_item *items, size_t count, void *stream);
/* dq8_linear with the projection's LoRA adapter (Projection::apply_quantized with
 * `adapter`, tensor.rs:134-183).  lora == NULL is dq8_linear. */
dq8_status dq8_linear_lora(dq8_ctx *ctx, const dq8_weights *w, const int8_t *q, const float *scales, size_t m,
                           const float *bias, const dq8_lora *lora, float *out, dq8_layout layout,
                           dq8_epilogue epilogue, void *stream);
/* dq8_linear_lora (lora may be NULL) in the rows layout whose stored result
 * out [m][n] is also quantized per token, as QuantizedInputs::new quantizes the
 * next projection's input (tensor.rs:315-353): q_out int8 [m][n] and scales_out
 * [m][ceil(n/64)].  This is the FFN's re-quantization of the SwiGlu product
 * before the down projection (qwen.rs:490-492).  A non-finite value in out is
 * reported as by dq8_quantize:
 * nonfinite == NULL synchronizes and returns DQ8_ERR_NONFINITE (q_out/scales_out
 * then unspecified; out is written); otherwise 1 is ORed into *nonfinite. */
dq8_status dq8_linear_q(dq8_ctx *ctx, const dq8_weights *w, const int8_t *q, const float *scales, size_t m,
                        const float *bias, const dq8_lora *lora, float *out, dq8_epilogue epilogue, int8_t *q_out,
                        float *scales_out, uint32_t *nonfinite, void *stream);
/* The weights of one layer's SwiGLU FFN (qwen.rs:486-492) and their optional
 * adapters.  gate/up adapters come with their middle products (dq8_lora_mid of
 * the FFN input x); the down adapter's middle product is computed from the
 * SwiGlu product h inside dq8_ffn, so its lora_A [rank][inter] is given instead. */
typedef struct dq8_ffn_weights {
    const dq8_weights *gate, *up, *down;  /* [inter][hidden], [inter][hidden], [hidden][inter] */
    const float *gate_bias, *up_bias, *down_bias;  /* NULL: +0.0 */
    const dq8_lora *gate_lora, *up_lora;           /* NULL: none */
    const float *down_lora_a, *down_lora_b;        /* NULL: none; [rank][inter], [hidden][rank] */
    size_t down_lora_rank;
    float down_lora_scale;
} dq8_ffn_weights;
/* The FFN's gate and up projections (qwen.rs:489-490) on one shared quantized
 * input: h = silu(gate(x) + gate_bias) * (up(x) + up_bias), exactly what
 * dq8_linear(gate, DQ8_WRITE into h) followed by dq8_linear(up, DQ8_SWIGLU
 * into h) store, bit for bit (Epilogue::SwiGlu, tensor.rs:96-99).  With more
 * than 64 rows both projections run in one launch that computes a gate and an
 * up tile of the same outputs side by side, so h is stored once and the gate
 * result is never written and read back.  No reference counterpart of its own:
 * it schedules the crate's two apply calls of the FFN together.  gate and up
 * must have the same shape; h is [m][n] (rows layout).
 * h_q/h_scales (both or neither; NULL: h is only stored): h is also quantized
 * for the down projection (qwen.rs:491, QuantizedInputs::new, tensor.rs:321-339)
 * into h_q [m][n] and h_scales [m][ceil(n/64)], exactly what dq8_quantize(h)
 * writes; on the one-launch path the launch itself does it, with no second
 * pass over h.  A non-finite value in h is reported as by dq8_quantize:
 * nonfinite == NULL synchronizes and returns DQ8_ERR_NONFINITE (h_q/h_scales
 * then unspecified; h is written); otherwise 1 is ORed into *nonfinite. */
dq8_status dq8_ffn_gate_up(dq8_ctx *ctx, const dq8_weights *gate, const dq8_weights *up, const int8_t *q,
                           const float *scales, size_t m, const float *gate_bias, const float *up_bias, float *h,
                           int8_t *h_q, float *h_scales, uint32_t *nonfinite, void *stream);
/* dq8_ffn_gate_up with the projections' LoRA adapters (either may be NULL):
 * the gate Write and up SwiGlu apply calls of Linear::apply_into_shared with
 * adapters (weights.rs:492-520; Adapter::combine, tensor.rs:109-117, after the
 * bias, tensor.rs:437-438), each adapter's middle product `mid` already
 * computed (dq8_lora_mid / dq8_lora_mid_batch).  The one-launch path takes
 * adapters of rank 0, and of rank 16 (the reference checkpoints' rank) with
 * 16-byte aligned mid and b: h is then still stored (and quantized) once.
 * Other adapters run as the two separate launches, with the same bits. */
dq8_status dq8_ffn_gate_up_lora(dq8_ctx *ctx, const dq8_weights *gate, const dq8_weights *up, const int8_t *q,
                                const float *scales, size_t m, const float *gate_bias, const float *up_bias,
                                const dq8_lora *gate_lora, const dq8_lora *up_lora, float *h, int8_t *h_q,
                                float *h_scales, uint32_t *nonfinite, void *stream);
/* One layer's FFN chain on the device (qwen.rs:486-492):
 *   h = gate(x)                          Write            (Linear::apply_shared)
 *   h = silu(h) * up(x)                  SwiGlu           (apply_into_shared)
 *   residual += down(h)                  Add, h re-quantized per token (apply_into)
 * q/scales are the FFN input's quantization, shared by gate and up (the
 * SharedInput of qwen.rs:488).  h [m][inter] is written (the crate's `gate`
 * buffer) and quantized on the device for down.  If h holds a non-finite
 * value, the down projection takes the crate's FP32 path (tensor.rs:197-201,
 * dq8_linear_fp32), chosen on the device: the call never synchronizes.  If
 * nonfinite is not NULL, 1 is ORed into *nonfinite when that happened. */
dq8_status dq8_ffn(dq8_ctx *ctx, const dq8_ffn_weights *f, const int8_t *q, const float *scales, size_t m, float *h,
                   float *residual, uint32_t *nonfinite, void *stream);
/* Projection::columns_tiled (tensor.rs:206-269), the FP32 path that
 * Projection::apply_quantized takes when QuantizedInputs::new(x) is None
 * (tensor.rs:197-201): for fp32 x [m][k], every output is
 *   y = dot_scores(x_r, w_n) + (bias[n] or 0.0),  w_n[t] = (float)q * scale
 * (Data::row, weights.rs:47-78), in dot_scores' x86-64 order (tensor.rs:6-25),
 * then the adapter term of Adapter::combine (lora may be NULL), stored through
 * the epilogue.  NaN and infinity propagate as in the crate. */
dq8_status dq8_linear_fp32(dq8_ctx *ctx, const dq8_weights *w, const float *x, size_t m, const float *bias,
                           const dq8_lora *lora, float *out, dq8_layout layout, dq8_epilogue epilogue,
                           void *stream);
/* Projection::apply_quantized (tensor.rs:127-202) on fp32 inputs x [m][k]:
 * quantize x (QuantizedInputs::new), then the int8 projection, or the FP32
 * path of dq8_linear_fp32 if x holds a non-finite value.  Both are queued and
 * a device flag lets exactly one run: no synchronization, the crate's result
 * either way.  Uses the context workspace (calls of one context are ordered). */
dq8_status dq8_apply(dq8_ctx *ctx, const dq8_weights *w, const float *x, size_t m, const float *bias,
                     const dq8_lora *lora, float *out, dq8_layout layout, dq8_epilogue epilogue, void *stream);
/* dq8_apply that allocates nothing, ever: no counterpart in the reference.  It
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * quantized inputs, their scales and the non-finite flag live in a fixed
 * 16 MiB device array of the library (one per GPU, held until the process
 * ends) instead of the context workspace: ceil(m*G*64/256)*256 +
 * ceil(m*ceil(G/4)*16/256)*256 bytes must fit in 16 MiB (G = ceil(k/64); for
 * example 2048 x 6144 or 4096 x 2048), else DQ8_ERR_LIMIT and nothing is
 * enqueued.  Results are those of dq8_apply, bit for bit.  All calls on one
 * GPU share that array, whatever their context: calls that overlap on one GPU
 * (two streams, or two host threads) race and give wrong results; each call's
 * flag is cleared by a kernel, so stream-ordered calls need no other care. */
dq8_status dq8_apply_noalloc(dq8_ctx *ctx, const dq8_weights *w, const float *x, size_t m, const float *bias,
                             const dq8_lora *lora, float *out, dq8_layout layout, dq8_epilogue epilogue,
                             void *stream);

/* Several independent projections in one launch (same-shape inputs are not
 * required).  Each item is one dq8_linear (or dq8_linear_lora).  This is the shape of a model
 * layer's projections that read already-available inputs (q/k/v, GDN
 * qkv/z/b/a, gate/up, or the continuation GEMMs of one question). */
typedef struct dq8_linear_item {
    const dq8_weights *w;
    const int8_t *q;      /* [m][k] int8 */
    const float *scales;  /* [m][G] */
    size_t m;
    const float *bias;    /* NULL: +0.0 */
    float *out;
    dq8_layout layout;
    dq8_epilogue epilogue;
    const dq8_lora *lora; /* NULL: no adapter */
} dq8_linear_item;
dq8_status dq8_linear_batch(dq8_ctx *ctx, const dq8_linear_item *items_host, size_t count, void *stream);

/* Debug: every per-group i32 dot, dots [m][n][G], computed by the same MFMA
 * path as dq8_linear (int8.rs:32-44 per group, as used at tensor.rs:429-436). */
dq8_status dq8_group_dots(dq8_ctx *ctx, const dq8_weights *w, const int8_t *q, size_t m, int32_t *dots,
                          void *stream);

/* Human-readable name of a status. */
const char *dq8_status_string(dq8_status s);

/* ---------------------------------------------------------------- safetensors
 * The checkpoint reader of read_tensors (weights.rs:298-365) over one file.
 * dq8_st_open reads and checks the header as read_tensors does with the
 * metadata rules of the safetensors crate 0.8.0 (Cargo.lock):
 *   - an 8-byte little-endian header size of at most 16 MiB, with the header
 *     inside the file;
 *   - a JSON object mapping tensor names to {"dtype", "shape", "data_offsets"},
 *     plus an optional "__metadata__" object of strings; a repeated key keeps
 *     its last value;
 *   - tensors ordered by data_offsets must tile the data section from 0
 *     without gaps or overlaps, each spanning exactly its shape's bytes;
 *   - the data section must end exactly at the end of the file.
 * Any violation returns DQ8_ERR_FORMAT (DQ8_ERR_IO if the file cannot be
 * read).  No tensor data is read by dq8_st_open.  Tensors are indexed in
 * file order (ascending data offsets, as Metadata::offset_keys).  Name, dtype
 * and shape pointers stay valid until dq8_st_close.  The host-only calls
 * (all but dq8_st_load_weights) need no GPU. */
typedef struct dq8_st dq8_st;
dq8_status dq8_st_open(const char *path, dq8_st **out);
dq8_status dq8_st_close(dq8_st *st);
dq8_status dq8_st_count(const dq8_st *st, size_t *count);
/* Tensor i: name, dtype as written in the file ("F32", "BF16", "I8", ...),
 * rank, shape and byte size. */
dq8_status dq8_st_info(const dq8_st *st, size_t i, const char **name, const char **dtype, size_t *ndim,
                       const size_t **shape, size_t *bytes);
/* Index of the tensor named `name` (DQ8_ERR_ARG if there is none). */
dq8_status dq8_st_find(const dq8_st *st, const char *name, size_t *index);
/* Data::read (weights.rs:147-195): tensor i's elements as stored, into host
 * memory dst of exactly its byte size.  Only F32, BF16 and F16 tensors can be
 * read (DQ8_ERR_FORMAT otherwise, "unsupported weight dtype"); a non-finite
 * element returns DQ8_ERR_NONFINITE ("non-finite weights"). */
dq8_status dq8_st_read_host(const dq8_st *st, size_t i, void *dst_host, size_t bytes);
/* Data::into_f32 (weights.rs:83-90) of tensor i into host memory: count must
 * equal its element count.  Same errors as dq8_st_read_host. */
dq8_status dq8_st_read_f32_host(const dq8_st *st, size_t i, float *dst_host, size_t count);
/* A projection weight (a 2-D F32/BF16/F16 tensor [n][k], k > 0, quantized at
 * load by weights.rs:346-355) straight from the file to a dq8_weights handle:
 * read into pinned staging, copied to the device, decoded, checked,
 * quantized and repacked there (dq8_weights_from_raw).  DQ8_ERR_SHAPE for
 * other ranks or k == 0. */
dq8_status dq8_st_load_weights(dq8_ctx *ctx, const dq8_st *st, size_t i, void *stream, dq8_weights **out);

#ifdef __cplusplus
}
#endif
#endif /* DQ8_H */

/*
 * dq8_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of decider-engine's `int8-compute` projection
 * arithmetic (Rust crate decider-engine 0.2.2).  It is the checker for the
 * HIP kernels and the CPU baseline that bench.py times; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library never links, loads or calls it, and it is not a fallback.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no fast-math, default
 * x86-64 target), so every float operation below is one IEEE-754 binary32
 * operation with round-to-nearest-even, as rustc emits for the cited Rust.
 *
 * Each function names the reference lines it restates.  Pinning (what checks
 * each function against something other than itself) is listed in the test
 * module tests/test_oracle.py; every function here is pinned there.
 */
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GROUP 64

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

/* weights.rs:120-125 and tensor.rs:330-335:
 *   max = fold(0.0, f32::max, |v|);  scale = max == 0 ? 1 : max(max / bound, f32::MIN_POSITIVE)
 * f32::max ignores a NaN operand exactly like fmaxf. */
static float group_scale(const float *v, size_t n, float bound) {
    float max = 0.0f;
    for (size_t i = 0; i < n; ++i) max = fmaxf(max, fabsf(v[i]));
    if (max == 0.0f) return 1.0f;
    return fmaxf(max / bound, FLT_MIN);
}

/* weights.rs:129 and tensor.rs:337: (v / scale).round().clamp(-b, b) as i8.
 * f32::round is half-away-from-zero (C roundf); clamp passes NaN through and
 * `as i8` maps NaN to 0 (saturating cast). */
static int8_t quantize_value(float v, float scale, float bound) {
    float r = roundf(v / scale);
    if (isnan(r)) return 0;
    if (r < -bound) r = -bound;
    if (r > bound) r = bound;
    return (int8_t)(int)r;
}

static void quantize_row(const float *row, size_t width, int8_t *q, float *scales) {
    size_t groups = div_ceil(width, GROUP);
    for (size_t g = 0; g < groups; ++g) {
        size_t start = g * GROUP;
        size_t n = width - start < GROUP ? width - start : GROUP;
        float s = group_scale(row + start, n, 127.0f);
        scales[g] = s;
        for (size_t i = 0; i < n; ++i) q[start + i] = quantize_value(row[start + i], s, 127.0f);
    }
}

/* ---------------------------------------------------------------- threads */

typedef void (*range_fn)(void *ctx, size_t begin, size_t end);
struct range_job { range_fn fn; void *ctx; size_t begin, end; };

static void *range_thread(void *arg) {
    struct range_job *j = (struct range_job *)arg;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

/* Split [0, n) into `threads` contiguous ranges.  Results never depend on the
 * split: every output element is computed by exactly one sequential loop, as
 * with rayon's par_chunks in the reference (tensor.rs:442-448). */
static void parallel_for(size_t n, int threads, range_fn fn, void *ctx) {
    if (threads <= 1 || n < 2) { fn(ctx, 0, n); return; }
    if ((size_t)threads > n) threads = (int)n;
    pthread_t tid[256];
    struct range_job jobs[256];
    if (threads > 256) threads = 256;
    size_t chunk = div_ceil(n, (size_t)threads);
    int launched = 0;
    for (int t = 0; t < threads; ++t) {
        size_t b = (size_t)t * chunk, e = b + chunk < n ? b + chunk : n;
        if (b >= e) break;
        jobs[t] = (struct range_job){fn, ctx, b, e};
        if (t == 0) continue;
        if (pthread_create(&tid[t], NULL, range_thread, &jobs[t]) != 0) { fn(ctx, b, e); jobs[t].fn = NULL; }
        launched = t + 1;
    }
    fn(ctx, jobs[0].begin, jobs[0].end);
    for (int t = 1; t < launched; ++t)
        if (jobs[t].fn) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------ quantizers */

struct qctx { const float *x; size_t width; int8_t *q; float *scales; };
static void quantize_rows_range(void *c, size_t b, size_t e) {
    struct qctx *q = (struct qctx *)c;
    size_t groups = div_ceil(q->width, GROUP);
    for (size_t r = b; r < e; ++r)
        quantize_row(q->x + r * q->width, q->width, q->q + r * q->width, q->scales + r * groups);
}

/* QuantizedInputs::new (tensor.rs:315-353).  Returns 1 (the reference's None)
 * when any element of the whole input is non-finite (tensor.rs:318-320), else
 * 0.  Rows run in parallel only when x.len() >= 65536 (tensor.rs:341). */
int dq8o_quantize_inputs(const float *x, size_t rows, size_t width, int8_t *q, float *scales, int threads) {
    size_t n = rows * width;
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(x[i])) return 1;
    struct qctx c = {x, width, q, scales};
    parallel_for(rows, n >= (1u << 16) ? threads : 1, quantize_rows_range, &c);
    return 0;
}

/* Data::quantize for 8 bits (weights.rs:98-146): per output row, per group of
 * 64, symmetric absmax to [-127, 127]; values are stored as u8 bit patterns
 * (weights.rs:131), scales row-major [rows][groups]. */
void dq8o_quantize_weights(const float *w, size_t rows, size_t width, uint8_t *values, float *scales) {
    size_t groups = div_ceil(width, GROUP);
    for (size_t r = 0; r < rows; ++r)
        quantize_row(w + r * width, width, (int8_t *)(values + r * width), scales + r * groups);
}

/* ------------------------------------------------------------------ dots */

/* scalar_dot (int8.rs:149-154); Kernel::dot asserts len <= 64 (int8.rs:33-36). */
int32_t dq8o_dot(const int8_t *a, const uint8_t *b, size_t len) {
    int32_t s = 0;
    for (size_t i = 0; i < len; ++i) s += (int32_t)a[i] * (int32_t)(int8_t)b[i];
    return s;
}

/* Kernel::scaled_dot (int8.rs:53-61): sum = 0.0; for each group in order,
 * sum += dot as f32 * (x_scale * w_scale) -- three rounded operations. */
float dq8o_scaled_dot(const int8_t *x, const float *xs, const uint8_t *w, const float *ws, size_t width) {
    float sum = 0.0f;
    size_t groups = div_ceil(width, GROUP);
    for (size_t g = 0; g < groups; ++g) {
        size_t start = g * GROUP;
        size_t n = width - start < GROUP ? width - start : GROUP;
        float p = xs[g] * ws[g];
        float t = (float)dq8o_dot(x + start, w + start, n) * p;
        sum = sum + t;
    }
    return sum;
}

/* Every per-group i32 dot, [rows][outputs][groups]: the "i32 accumulators" of
 * the path (int8.rs:32-44 applied per group as in tensor.rs:429-436). */
void dq8o_group_dots(const int8_t *q, size_t rows, const uint8_t *w, size_t outputs, size_t width, int32_t *dots) {
    size_t groups = div_ceil(width, GROUP);
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < outputs; ++c)
            for (size_t g = 0; g < groups; ++g) {
                size_t start = g * GROUP;
                size_t n = width - start < GROUP ? width - start : GROUP;
                dots[(r * outputs + c) * groups + g] = dq8o_dot(q + r * width + start, w + c * width + start, n);
            }
}

/* ---------------------------------------------------------- linear_int8 */

struct lctx {
    const int8_t *q; const float *xs; size_t rows;
    const uint8_t *w; const float *ws; size_t width;
    const float *bias; float *columns;
};
/* The per-column closure of linear_int8 (tensor.rs:415-440) without adapter:
 * for every row, scaled_dot then `sum + bias` with bias 0.0 when absent (437). */
static void linear_columns_range(void *c, size_t b, size_t e) {
    struct lctx *l = (struct lctx *)c;
    size_t groups = div_ceil(l->width, GROUP);
    for (size_t col = b; col < e; ++col) {
        const uint8_t *w = l->w + col * l->width;
        const float *ws = l->ws + col * groups;
        float bias = l->bias ? l->bias[col] : 0.0f;
        for (size_t r = 0; r < l->rows; ++r) {
            float sum = dq8o_scaled_dot(l->q + r * l->width, l->xs + r * groups, w, ws, l->width);
            l->columns[col * l->rows + r] = sum + bias;
        }
    }
}

/* linear_int8 (tensor.rs:379-456) on already-quantized inputs: output columns
 * are column-major [outputs][rows]; columns run in parallel when
 * rows * outputs >= 512 (tensor.rs:442). */
void dq8o_linear_int8(const int8_t *q, const float *xs, size_t rows, const uint8_t *w, const float *ws,
                      size_t outputs, size_t width, const float *bias, float *columns, int threads) {
    struct lctx c = {q, xs, rows, w, ws, width, bias, columns};
    parallel_for(outputs, rows * outputs >= 512 ? threads : 1, linear_columns_range, &c);
}

/* qwen.rs:194-199: silu(x) = x * sigmoid(x), sigmoid(x) = 1 / (1 + exp(-x));
 * f32::exp lowers to the platform libm expf. */
float dq8o_silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

struct sctx { const float *x; float *y; };
static void silu_range(void *c, size_t b, size_t e) {
    struct sctx *s = (struct sctx *)c;
    for (size_t i = b; i < e; ++i) s->y[i] = dq8o_silu(s->x[i]);
}
/* dq8o_silu over an array. */
void dq8o_silu_n(const float *x, float *y, size_t n, int threads) {
    struct sctx c = {x, y};
    parallel_for(n, n >= (1u << 16) ? threads : 1, silu_range, &c);
}

/* The algorithm of the libm expf that f32::exp lowers to on the reference's
 * platform: glibc 2.35 on x86-64 (sysdeps/ieee754/flt-32/e_expf.c, from ARM's
 * optimized-routines), in the form of glibc's FMA build (__expf_fma, chosen on
 * every x86-64 with FMA3).  With n = 32 and InvLn2N = n / ln 2:
 *   kd = fma(InvLn2N, x, 1.5*2^52)  -> low bits of kd hold k = round(x n/ln2)
 *   r  = fma(InvLn2N, x, -(kd - 1.5*2^52))
 *   s  = 2^(k/n) from a table of 2^(j/n), j = k mod n, and the exponent k div n
 *   y  = fma(fma(c0, r, c1), r*r, fma(c2, r, 1)) * s, rounded once to float,
 * with c0..c2 the cubic's coefficients for 2^(r/n).  x >= 89 overflows to
 * +inf, x <= -104 gives +0, NaN returns x + x.  The kernels restate the same
 * steps; dq8o_silu itself calls libm expf.  Pinned against the host expf on
 * every binary32 input (dq8o_expf_mismatches). */
static uint64_t exp2_frac_bits[32];
static pthread_once_t exp2_frac_once = PTHREAD_ONCE_INIT;
static void exp2_frac_init(void) {
    for (int j = 0; j < 32; ++j) {
        double v = exp2((double)j / 32.0);
        memcpy(&exp2_frac_bits[j], &v, 8);
    }
}
float dq8o_expf_restated(float x) {
    if (x != x) return x + x;
    if (x >= 89.0f) return INFINITY;
    if (x <= -104.0f) return 0.0f;
    pthread_once(&exp2_frac_once, exp2_frac_init);
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    uint64_t j = ki & 31u, sb = exp2_frac_bits[j] + ((ki - j) << 47);
    double s;
    memcpy(&s, &sb, 8);
    double z = fma(c0, r, c1), r2 = r * r, y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

struct ectx { uint64_t base; size_t mismatches; };
static void expf_range(void *c, size_t b, size_t e) {
    struct ectx *x = (struct ectx *)c;
    size_t bad = 0;
    for (size_t i = b; i < e; ++i) {
        uint32_t bits = (uint32_t)(x->base + i);
        float v, want, got;
        memcpy(&v, &bits, 4);
        want = expf(v);
        got = dq8o_expf_restated(v);
        bad += memcmp(&want, &got, 4) != 0;
    }
    __atomic_fetch_add(&x->mismatches, bad, __ATOMIC_RELAXED);
}
/* Number of binary32 bit patterns in [begin, end) (end <= 2^32) where
 * dq8o_expf_restated differs in any bit from the host libm expf. */
size_t dq8o_expf_mismatches(uint64_t begin, uint64_t end, int threads) {
    if (end > (1ull << 32)) end = 1ull << 32;
    if (end <= begin) return 0;
    struct ectx c = {begin, 0};
    pthread_once(&exp2_frac_once, exp2_frac_init);
    parallel_for((size_t)(end - begin), threads, expf_range, &c);
    return c.mismatches;
}

/* write_columns (tensor.rs:272-288) with Epilogue::store (tensor.rs:92-99):
 * 0 Write (dst = v), 1 Add (dst += v), 2 SwiGlu (dst = silu(dst) * v). */
void dq8o_write_columns(const float *columns, size_t rows, size_t outputs, float *result, int epilogue) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < outputs; ++c) {
            float v = columns[c * rows + r];
            float *dst = result + r * outputs + c;
            if (epilogue == 0) *dst = v;
            else if (epilogue == 1) *dst = *dst + v;
            else *dst = dq8o_silu(*dst) * v;
        }
}

/* The x86 (non-SDOT) plan of Linear::apply_into_shared (weights.rs:450-491)
 * without LoRA: `linear` re-quantizes its input (tensor.rs:404), computes the
 * int8 columns and writes them through the epilogue.  Returns 1 where the
 * reference falls back to FP32 (non-finite input), leaving `result` as is. */
int dq8o_linear(const float *x, size_t rows, size_t width, const uint8_t *w, const float *ws, size_t outputs,
                const float *bias, float *result, int epilogue, int threads) {
    if (rows == 0) return 0;
    size_t groups = div_ceil(width, GROUP);
    size_t nq = rows * width, ns = rows * groups, nc = rows * outputs;
    int8_t *q = (int8_t *)malloc(nq > 0 ? nq : 1);
    float *xs = (float *)malloc((ns > 0 ? ns : 1) * sizeof(float));
    float *columns = (float *)malloc((nc > 0 ? nc : 1) * sizeof(float));
    int status = 2;
    if (q && xs && columns) {
        status = dq8o_quantize_inputs(x, rows, width, q, xs, threads);
        if (status == 0) {
            dq8o_linear_int8(q, xs, rows, w, ws, outputs, width, bias, columns, threads);
            dq8o_write_columns(columns, rows, outputs, result, epilogue);
        }
    }
    free(q); free(xs); free(columns);
    return status;
}

/* -------------------------------------------------------------- LoRA (FP32) */

/* dot_scores (tensor.rs:6-25), the x86-64 branch: eight partial sums, element i
 * of every 8-element chunk going to lane i % 8 as `lane += a * b` (a rounded
 * product, then a rounded add: Rust does not contract on x86-64); the lanes are
 * summed in order by f32::sum, whose fold starts at -0.0; then the tail
 * (len % 8 elements) is added one product at a time. */
float dq8o_dot_scores(const float *a, const float *b, size_t len) {
    size_t chunks = len / 8;
    float lanes[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t c = 0; c < chunks; ++c)
        for (int i = 0; i < 8; ++i) {
            float p = a[8 * c + i] * b[8 * c + i];
            lanes[i] = lanes[i] + p;
        }
    float sum = -0.0f;
    for (int i = 0; i < 8; ++i) sum = sum + lanes[i];
    for (size_t t = 8 * chunks; t < len; ++t) {
        float p = a[t] * b[t];
        sum = sum + p;
    }
    return sum;
}

struct fctx {
    const float *x; size_t rows; size_t width;
    const float *w; const float *bias; float *columns;
};
/* The x86 FP32 columns (Projection::columns_tiled with T = 1, tensor.rs:206-269)
 * without adapter: column j, row r = dot_scores(x_r, w_j) + bias[j], the bias
 * being 0.0 when absent (tensor.rs:247-250). */
static void fp32_columns_range(void *c, size_t b, size_t e) {
    struct fctx *f = (struct fctx *)c;
    for (size_t col = b; col < e; ++col) {
        float bias = f->bias ? f->bias[col] : 0.0f;
        for (size_t r = 0; r < f->rows; ++r)
            f->columns[col * f->rows + r] = dq8o_dot_scores(f->x + r * f->width, f->w + col * f->width, f->width) + bias;
    }
}

/* `linear` (tensor.rs:290-307) of an FP32 weight matrix w [outputs][width] with
 * Epilogue::Write: result [rows][outputs].  Columns run in parallel when
 * rows * outputs >= 512 (tensor.rs:254); results do not depend on it. */
void dq8o_linear_f32(const float *x, size_t rows, size_t width, const float *w, size_t outputs, const float *bias,
                     float *result, int threads) {
    size_t nc = rows * outputs;
    if (nc == 0) return;
    float *columns = (float *)malloc(nc * sizeof(float));
    if (!columns) return;
    struct fctx c = {x, rows, width, w, bias, columns};
    parallel_for(outputs, nc >= 512 ? threads : 1, fp32_columns_range, &c);
    dq8o_write_columns(columns, rows, outputs, result, 0);
    free(columns);
}

/* The LoRA middle product of Linear::apply_into_shared (weights.rs:480 and
 * 495): mid [rows][rank] = linear(x, A) with A [rank][width], no bias. */
void dq8o_lora_mid(const float *x, size_t rows, size_t width, const float *a, size_t rank, float *mid, int threads) {
    dq8o_linear_f32(x, rows, width, a, rank, NULL, mid, threads);
}

/* Adapter::combine (tensor.rs:109-117): base + scale * (dot_scores(mid_row,
 * b_row) + 0.0), the multiply and the add rounded separately. */
float dq8o_lora_combine(float base, const float *mid_row, const float *b_row, size_t rank, float scale) {
    float delta = dq8o_dot_scores(mid_row, b_row, rank) + 0.0f;
    float scaled = scale * delta;
    return base + scaled;
}

int dq8o_linear_lora(const float *x, size_t rows, size_t width, const uint8_t *w, const float *ws, size_t outputs,
                     const float *bias, const float *a, const float *b, size_t rank, float scale, float *result,
                     int epilogue, int threads);
/* Data::row of 8-bit Quantized data (weights.rs:47-78): element i of row r is
 * (float)(int8)values[r][i] * scales[r][i / 64], one rounding. */
void dq8o_dequantize_weights(const uint8_t *w, const float *ws, size_t n, size_t k, float *out) {
    size_t g = div_ceil(k, GROUP);
    for (size_t r = 0; r < n; ++r)
        for (size_t i = 0; i < k; ++i) out[r * k + i] = (float)(int8_t)w[r * k + i] * ws[r * g + i / GROUP];
}

/* Projection::apply_quantized (tensor.rs:127-202) with its FP32 fallback: if
 * QuantizedInputs::new(x) is None (a non-finite input), the columns are
 * columns_tiled (tensor.rs:206-269) over the dequantized weights --
 * dot_scores(x_r, w_n) + bias -- and the adapter (a != NULL) adds
 * scale * (dot_scores(mid_r, b_n) + 0.0) with mid = linear(x, A); otherwise the
 * int8 path of dq8o_linear_lora / dq8o_linear.  Stores through the epilogue.
 * Returns 1 if the FP32 path ran, 0 if the int8 path did, 2 on allocation failure. */
int dq8o_apply(const float *x, size_t rows, size_t width, const uint8_t *w, const float *ws, size_t outputs,
               const float *bias, const float *a, const float *b, size_t rank, float scale, float *result,
               int epilogue, int threads) {
    if (rows == 0) return 0;
    int st = a ? dq8o_linear_lora(x, rows, width, w, ws, outputs, bias, a, b, rank, scale, result, epilogue, threads)
               : dq8o_linear(x, rows, width, w, ws, outputs, bias, result, epilogue, threads);
    if (st != 1) return st;
    size_t nv = rows * outputs, nm = rows * rank;
    float *deq = (float *)malloc((outputs * width > 0 ? outputs * width : 1) * sizeof(float));
    float *values = (float *)malloc((nv > 0 ? nv : 1) * sizeof(float));
    float *mid = (float *)malloc((nm > 0 ? nm : 1) * sizeof(float));
    float *delta = (float *)malloc((nv > 0 ? nv : 1) * sizeof(float));
    int status = 2;
    if (deq && values && mid && delta) {
        dq8o_dequantize_weights(w, ws, outputs, width, deq);
        dq8o_linear_f32(x, rows, width, deq, outputs, bias, values, threads);
        if (a) {
            dq8o_lora_mid(x, rows, width, a, rank, mid, threads);
            dq8o_linear_f32(mid, rows, rank, b, outputs, NULL, delta, threads);
            for (size_t i = 0; i < nv; ++i) {
                float scaled = scale * delta[i];
                values[i] = values[i] + scaled;
            }
        }
        for (size_t i = 0; i < nv; ++i) {
            if (epilogue == 0) result[i] = values[i];
            else if (epilogue == 1) result[i] = result[i] + values[i];
            else result[i] = dq8o_silu(result[i]) * values[i];
        }
        status = 1;
    }
    free(deq); free(values); free(mid); free(delta);
    return status;
}

/* The x86 (non-SDOT) plan of Linear::apply_into_shared with a LoRA pair
 * (weights.rs:450-491): values = linear(x, W, bias) (the int8 projection);
 * mid = linear(x, A); delta = linear(mid, B); values[i] += scale * delta[i];
 * then the epilogue stores values into result.  A is [rank][width] and B is
 * [outputs][rank], both FP32.  Returns 1 where the reference falls back to FP32
 * for the base projection (non-finite input), leaving `result` as is. */
int dq8o_linear_lora(const float *x, size_t rows, size_t width, const uint8_t *w, const float *ws, size_t outputs,
                     const float *bias, const float *a, const float *b, size_t rank, float scale, float *result,
                     int epilogue, int threads) {
    if (rows == 0) return 0;
    size_t nv = rows * outputs, nm = rows * rank;
    float *values = (float *)malloc((nv > 0 ? nv : 1) * sizeof(float));
    float *mid = (float *)malloc((nm > 0 ? nm : 1) * sizeof(float));
    float *delta = (float *)malloc((nv > 0 ? nv : 1) * sizeof(float));
    int status = 2;
    if (values && mid && delta) {
        status = dq8o_linear(x, rows, width, w, ws, outputs, bias, values, 0, threads);
        if (status == 0) {
            dq8o_lora_mid(x, rows, width, a, rank, mid, threads);
            dq8o_linear_f32(mid, rows, rank, b, outputs, NULL, delta, threads);
            for (size_t i = 0; i < nv; ++i) {
                float scaled = scale * delta[i];
                values[i] = values[i] + scaled;
            }
            for (size_t i = 0; i < nv; ++i) {
                if (epilogue == 0) result[i] = values[i];
                else if (epilogue == 1) result[i] = result[i] + values[i];
                else result[i] = dq8o_silu(result[i]) * values[i];
            }
        }
    }
    free(values); free(mid); free(delta);
    return status;
}

/*
 * jevons_qmm.h — C ABI of the MI355X (gfx950) quantized GGML matrix products.
 *
 * Drop-in boundary for jevons-rs's quantized matmul path. Each entry point names the reference
 * interface it replaces (paths relative to the reference repository root):
 *   crates/jevons-kernels/src/gemm.rs        QMatrix, Plan, SplitScratch, matmul*, matvec
 *   crates/jevons-kernels/src/lib.rs         Gpu (device client), Buf (device buffer + length)
 *   crates/jevons-formats/src/gguf.rs        TensorType ids and block sizes
 *   crates/jevons-burn/src/kernels.rs        GemmOps::f16_matmul (Burn operator)
 *   crates/jevons-core/src/model.rs          greedy (argmax of a logit row)
 *
 * Conventions
 *  - Every call returns a jv_status; JV_OK is 0. On failure jv_last_error() returns a message
 *    for the calling thread that names the type and shape like the reference's Err strings.
 *    Nothing aborts; bad shapes and short buffers are rejected on the host (the reference's
 *    launch asserts and CubeCL checked launches, gemm.rs:1137, :1172, :1218, :1285).
 *  - Buffers passed to products are device pointers with a logical length in elements (the
 *    reference's Buf length, lib.rs:76-124). Products are asynchronous on `stream`
 *    (a hipStream_t; NULL is the default stream). jv_sync waits for the device.
 *  - A jv_ctx is used from one host thread at a time (the reference's API is not Sync).
 *  - Outputs are out[r, c] = sum_k x[r, k] * W[c, k] accumulated in fp32.
 */
#ifndef JEVONS_QMM_H
#define JEVONS_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    JV_OK = 0,
    JV_ERR_INVALID = 1,     /* bad argument, shape or length */
    JV_ERR_UNSUPPORTED = 2, /* tensor type or encoding without a GPU layout */
    JV_ERR_HIP = 3,         /* the HIP runtime reported an error */
    JV_ERR_NO_KERNELS = 4,  /* the gfx950 code object could not be loaded */
    JV_ERR_NO_MEMORY = 5    /* device allocation failed */
} jv_status;

/* Kernel weight encodings; values equal FMT_* (gemm.rs:25-30). */
typedef enum { JV_FMT_Q4K = 0, JV_FMT_Q6K = 1, JV_FMT_Q5_0 = 2, JV_FMT_Q8_0 = 3, JV_FMT_F16 = 4 } jv_fmt;

/* GGML tensor type ids (TensorType::from_id, gguf.rs:120-131). */
enum {
    JV_GGML_F32 = 0, JV_GGML_F16 = 1, JV_GGML_Q5_0 = 6, JV_GGML_Q8_0 = 8, JV_GGML_Q4K = 12,
    JV_GGML_Q6K = 14
};

/* Activation element type. The reference takes FP16 rows (gemm.rs:405, :537); BF16 and F32
 * rows are converted to FP16 on chip (exact for BF16 magnitudes in [2^-14, 65504]; F32 rounds to
 * nearest even, as the reference's upload_f16 does). A row holding values beyond the FP16 range
 * is first divided by a power of two and its outputs multiplied back, which is exact (the
 * reference's f16_linear_scaled rule, crates/jevons-burn/src/kernels.rs:105, :120-130, with a
 * power of two): tiled products scale rows whose largest magnitude exceeds 16384, small-row
 * products the columns of a row in which some value overflowed FP16. Values far below the row's
 * largest then lose low bits, as FP16 subnormals. */
typedef enum { JV_ACT_F16 = 0, JV_ACT_BF16 = 1, JV_ACT_F32 = 2 } jv_act;

/* Output element type. The reference writes FP32; BF16 rounds the FP32 sum to nearest even. */
typedef enum { JV_OUT_F32 = 0, JV_OUT_BF16 = 1 } jv_out;

/* Launch plan (Plan, gemm.rs:973-979): bm == 0 selects the small-row product (m <= 16).
 * bm in {32, 64, 128} rows, bn in {64, 128} columns as the reference allows, plus bn = 256
 * on gfx950; splits in 1..=16 divides K (partials summed in a fixed order). */
typedef struct {
    uint32_t bm, bn, splits;
} jv_plan;

typedef struct jv_ctx jv_ctx;         /* Gpu (lib.rs:17-306) */
typedef struct jv_qmatrix jv_qmatrix; /* QMatrix (gemm.rs:817-829) */
typedef struct jv_scratch jv_scratch; /* SplitScratch (gemm.rs:1041-1065) */

typedef struct {
    int device;
    int compute_units;
    int wave_size;
    size_t lds_bytes;       /* LDS per workgroup */
    size_t total_memory;
    char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} jv_device_info;

/* (elements, bytes) per block of a GGML type id; JV_ERR_UNSUPPORTED for other ids
 * (TensorType::block, gguf.rs:134-144). */
jv_status jv_type_block(uint32_t ggml_type, uint32_t *elems, uint32_t *bytes);

/* Opens HIP device `device` and loads the gfx950 code object (Gpu::new, lib.rs:181-197).
 * The code object is looked up in $JV_CODE_OBJECT, else next to this library. Like the
 * reference's Gpu (one queue, not Sync), a context serves one host thread at a time, and its
 * products run in the order they are queued: the context's own staging buffers (packed
 * activations; split-K counters and partials of jv_matvec) are reused by every product, so
 * products of one context must not run concurrently on different streams. */
jv_status jv_open(int device, jv_ctx **out);
void jv_close(jv_ctx *ctx);
jv_status jv_device_info_get(jv_ctx *ctx, jv_device_info *info);
/* Waits for all queued work on the context's device (Gpu::sync, lib.rs:294-302). */
jv_status jv_sync(jv_ctx *ctx);

/* Uploads GGML blocks of `ggml_type` for weights [experts * n, k] (QMatrix::upload,
 * gemm.rs:822-841). `raw` is host memory of exactly experts*n*k/block*size bytes. The blocks
 * are repacked on the device into the gfx950 layout; decoded values are unchanged. */
jv_status jv_qmatrix_upload(jv_ctx *ctx, uint32_t ggml_type, size_t n, size_t k, size_t experts,
                            const void *raw, size_t bytes, jv_qmatrix **out);
/* Same, with `raw_dev` already in device memory (no host copy). */
jv_status jv_qmatrix_upload_device(jv_ctx *ctx, uint32_t ggml_type, size_t n, size_t k,
                                   size_t experts, const void *raw_dev, size_t bytes,
                                   jv_qmatrix **out);
/* Uploads the reference's packed regions (QMatrix::from_packed, gemm.rs:844-899; region
 * sizes per quant::packed_words, quant.rs:127-135). Packed scales must be FP16 values. */
jv_status jv_qmatrix_from_packed(jv_ctx *ctx, uint32_t ggml_type, size_t n, size_t k,
                                 size_t experts, const uint32_t *q, size_t nq, const uint32_t *h,
                                 size_t nh, const uint32_t *s, size_t ns, const float *d,
                                 size_t nd, jv_qmatrix **out);
/* Views caller-owned row-major FP16 device weights [n, k] stored as n*k/2 words without a copy
 * (QMatrix::f16_view / from_f16_words, gemm.rs:903-948). The caller keeps the buffer alive. */
jv_status jv_qmatrix_f16_view(jv_ctx *ctx, size_t n, size_t k, const void *dev_words,
                              size_t words, jv_qmatrix **out);
void jv_qmatrix_free(jv_qmatrix *w);
/* Device bytes held by the matrix (QMatrix::bytes, gemm.rs:950-952). */
size_t jv_qmatrix_bytes(const jv_qmatrix *w);
jv_status jv_qmatrix_shape(const jv_qmatrix *w, uint32_t *fmt, size_t *n, size_t *k,
                           size_t *experts);

/* Plan::heuristic (gemm.rs:987-1004), unchanged: row-invariant plans never split K or use the
 * small-row kernel; `groups_target` is the workgroup count that fills the device. */
jv_plan jv_plan_heuristic(const jv_qmatrix *w, size_t m, int row_invariant, size_t groups_target);
/* The plan this library picks for gfx950 (256 compute units) when none is given. */
jv_plan jv_plan_auto(const jv_qmatrix *w, size_t m, int row_invariant);
/* Plan::valid_for (gemm.rs:1006-1015), plus bn = 256. Returns 1 if valid, 0 if not. */
int jv_plan_valid(const jv_qmatrix *w, size_t m, jv_plan plan);

/* Grow-on-demand split-K partial buffer (SplitScratch, gemm.rs:1041-1065). */
jv_status jv_scratch_new(jv_ctx *ctx, jv_scratch **out);
void jv_scratch_free(jv_scratch *s);

/* out[m, n] = x[m, k] . W^T with this library's plan (matmul, gemm.rs:1069-1088). A plan that
 * splits K stages its partials in `scratch`, or in a buffer the context owns when it is null. */
jv_status jv_matmul(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                    const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                    jv_scratch *scratch, void *stream);
/* Bytes of the fixed device array of jv_matmul_noalloc, one per GPU: 256 KiB of split-K tile
 * counters, then the staging payload. */
#define JV_NOALLOC_SCRATCH_BYTES (32u << 20)

/* No counterpart in the reference. For callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. The product and its
 * kernels are jv_matmul's with a scratch buffer, but every staging buffer (packed activations of
 * the tiled products, split-K partials and tile counters) lives in one fixed device array of
 * JV_NOALLOC_SCRATCH_BYTES per GPU, set up by jv_open. The call allocates and frees no memory.
 * A split-K tile plan whose staging would not fit runs with whole K on the same tile instead
 * (then its bits can differ from jv_matmul's, within the products' accuracy). A product that
 * still needs more staging than the array holds is rejected with JV_ERR_INVALID (the
 * message names the bytes needed and the limit). All calls on one GPU share that GPU's array,
 * which keeps the last call's contents: calls that overlap on one GPU (on other streams, or from
 * other contexts or threads) race. */
jv_status jv_matmul_noalloc(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                            const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                            void *stream);
/* Product with an explicit plan (matmul_plan, gemm.rs:1093-1119). Plans with splits == 1 are
 * row invariant: every output row is accumulated in the same order whatever m or the tile. */
jv_status jv_matmul_plan(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                         const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                         jv_scratch *scratch, jv_plan plan, void *stream);
/* Small-row product, m <= 16 (matvec, gemm.rs:1136-1168). */
jv_status jv_matvec(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                    const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                    void *stream);
/* Tiled product with split-K (matmul_split, gemm.rs:1206-1257; matmul_tiled :1122-1133 is
 * splits = 1). `scratch` may be NULL when splits == 1. */
jv_status jv_matmul_split(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                          const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                          uint32_t bm, uint32_t bn, uint32_t splits, jv_scratch *scratch,
                          void *stream);

/* Expert grouping produced on the device (Groups, gemm.rs:955-966): sorted assignment ids,
 * per-expert offsets [experts + 1] and jobs (jobs[0] = count, then (expert, start) pairs), all
 * device uint32 buffers; max_jobs bounds the job count (the grid); input row = id / in_div;
 * rows = output rows (assignments). */
typedef struct {
    const uint32_t *ids;
    const uint32_t *offsets;
    const uint32_t *jobs;
    size_t max_jobs;
    uint32_t in_div;
    size_t rows;
} jv_groups;

/* Expert grouping of routed assignments (ops::group_routes / group,
 * crates/jevons-gemma4-diffusion/src/gpu/ops.rs:1100-1130 and :522-587): device ids
 * [assignments] -> sorted [assignments], offsets [experts + 1], jobs [jobs_len] for row tiles
 * of bm. Ids >= experts are not routed. experts <= 1024; jobs_len must hold
 * 1 + 2 * (ceil(assignments / bm) + experts) words. */
jv_status jv_group_routes(jv_ctx *ctx, const uint32_t *ids, size_t assignments, size_t experts,
                          uint32_t bm, uint32_t *sorted, uint32_t *offsets, uint32_t *jobs,
                          size_t jobs_len, void *stream);
/* Expert-grouped product (matmul_grouped, gemm.rs:1274-1321): job j multiplies up to bm sorted
 * rows of expert e by that expert's weight rows [e n, (e + 1) n) and writes output rows ids[s]
 * of out [g.rows, n]. bm in {16, 32, 64, 128}, bn in {64, 128, 256}; splits > 1 divides K and
 * sums the partials in `scratch`. */
jv_status jv_matmul_grouped(jv_ctx *ctx, const void *x, jv_act act, size_t x_len,
                            const jv_qmatrix *w, const jv_groups *g, void *out, jv_out out_type,
                            size_t out_len, uint32_t bm, uint32_t bn, uint32_t splits,
                            jv_scratch *scratch, void *stream);
/* Expert-grouped small-row product (matvec_grouped, gemm.rs:1171-1203): jobs of at most
 * mr <= 16 rows. */
jv_status jv_matvec_grouped(jv_ctx *ctx, const void *x, jv_act act, size_t x_len,
                            const jv_qmatrix *w, const jv_groups *g, void *out, jv_out out_type,
                            size_t out_len, uint32_t mr, void *stream);

/* Burn operator GemmOps::f16_matmul (crates/jevons-burn/src/kernels.rs:52-97): dense row-major
 * FP16 x [m, k] times FP16 weight [n, k]^T into FP32 out [m, n], with the row-invariant plan
 * rule of kernels.rs:16-31. n and k must be multiples of 64. */
jv_status jv_f16_matmul(jv_ctx *ctx, const void *x, size_t m, size_t k, const void *weight,
                        size_t n, float *out, void *stream);

/* Per-row argmax of FP32 logits [rows, n] with greedy's rule (model.rs:207-219): the first
 * maximum wins; a row holding a non-finite value or n == 0 yields index -1. `index` is a
 * device buffer of `rows` int32. `scratch` holds the per-chunk partials. */
jv_status jv_argmax_rows(jv_ctx *ctx, const float *logits, size_t rows, size_t n,
                         int32_t *index, jv_scratch *scratch, void *stream);

/* The vocabulary projection with its soft cap and greedy's argmax in one call (the full-logits
 * forward, crates/jevons-gemma4-diffusion/src/model.rs:1192-1204: matmul, then softcap_logits;
 * then greedy per row, crates/jevons-core/src/model.rs:180-187, :207-219): out [m, n] FP32 =
 * x . W^T on jv_matmul's plan, soft-capped in place when cap > 0 (cap = 0: raw logits), and
 * index[r] (device, m int32) = greedy's argmax of out row r (-1 for a row holding a non-finite
 * value). The results equal jv_matmul, jv_softcap_logits and jv_argmax_rows in turn. The
 * persistent small-row kernels and the Q4_K / Q6_K / Q8_0 register tiles (whole K) soft-cap
 * their outputs and fold each row's maximum into a per-row key of the context as they store,
 * and a small second launch writes `index` from the keys, so the logits are not read again;
 * other kernels are followed by the two other steps (which use `scratch`). The context's key
 * buffer grows on the first call with more rows than before (run each row count once before
 * graph capture), and calls on one context must not run concurrently (they share the keys).
 * m <= 65535. */
jv_status jv_matmul_argmax(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                           const jv_qmatrix *w, float *out, size_t out_len, float cap, int32_t *index,
                           jv_scratch *scratch, void *stream);

/* Final-logit soft capping in place (softcap_logits, crates/jevons-gemma4-diffusion/src/gpu/
 * ops.rs:1159-1168, kernel :750-758): x[i] = cap * tanh(x[i] / cap) for i < len; cap > 0. */
jv_status jv_softcap_logits(jv_ctx *ctx, float *x, size_t len, float cap, void *stream);
/* Candidate logits (pick, gpu/ops.rs:1133-1157, kernel pick_logits :589-634): for each of
 * `count` device (row, token) pairs, out[p] = cap * tanh(x[row] . E[token] / cap), with E the
 * weight rows of `table` (K = d, decoded exactly) and x [x_len / d][d]. A pair naming a row or
 * token out of range gives NaN. */
jv_status jv_pick_logits(jv_ctx *ctx, const void *x, jv_act act, size_t x_len,
                         const jv_qmatrix *table, const uint32_t *pairs, size_t count, float *out,
                         size_t out_len, float cap, void *stream);

/* Exactness probes: decode rows [row0, row0 + rows) of `w` with the products' own device
 * decoder into FP32 (equal to quant::dequantize, quant.rs:83-101) or FP16 (the on-chip weight
 * tile, round-to-nearest-even of that FP32 value). Outputs are device [rows, k]. */
jv_status jv_dequant_rows_f32(jv_ctx *ctx, const jv_qmatrix *w, size_t row0, size_t rows,
                              float *out, void *stream);
jv_status jv_dequant_rows_f16(jv_ctx *ctx, const jv_qmatrix *w, size_t row0, size_t rows,
                              uint16_t *out, void *stream);

/* ---------------------------------------------------------------------------------------------
 * Launch-plan tuner and its table (crates/jevons-gemma4-diffusion/src/gpu/tune.rs). Plans are
 * keyed by (format, n, k, row bucket, row invariance) and, for grouped products, (format, n, k,
 * experts, row bucket); a bucket b = max(next power of two of m, 4) serves m in (b/2, b]
 * (tune.rs:73-76). Lookups fall back to jv_plan_auto (grouped: bm 32, bn 128 or 64); a stored
 * row-invariant plan is used only if it splits no K (tune.rs:162-174, :485-487).
 * ------------------------------------------------------------------------------------------ */
typedef struct jv_tuner jv_tuner;
/* Row bucket of m (tune.rs:73-76). */
size_t jv_tune_bucket(size_t m);
/* Buckets tuned for row counts up to `max` from `min` (buckets, tune.rs:489-497): min, 2 min, ...
 * up to bucket(max) and at most 1024. Writes up to `cap` of them; returns their count. */
size_t jv_tune_buckets(size_t min, size_t max, size_t *out, size_t cap);
/* The measured plan rule (pick, tune.rs:556-566): index of the fastest of n timed candidates,
 * unless it beats the candidate whose id is `baseline` by less than 5%; -1 if n == 0. */
int jv_tune_pick(const double *times, const uint32_t *ids, size_t n, uint32_t baseline);
/* Tuner for this context's device (Tuner::new, tune.rs:132-151): loads `path` (NULL: nothing
 * stored) when its profile line matches the device. */
jv_status jv_tuner_new(jv_ctx *ctx, const char *path, jv_tuner **out);
/* A table without a device (lookups and storage only), for the given profile line. */
jv_status jv_tuner_open_table(const char *profile, const char *path, jv_tuner **out);
void jv_tuner_free(jv_tuner *t);
const char *jv_tuner_profile(const jv_tuner *t);
size_t jv_tuner_entries(const jv_tuner *t);
/* Stored dense plan for (fmt, n, k, bucket(m), row_invariant); 1 if present. */
int jv_tuner_lookup_dense(const jv_tuner *t, uint32_t fmt, size_t n, size_t k, size_t m,
                          int row_invariant, jv_plan *plan);
void jv_tuner_insert_dense(jv_tuner *t, uint32_t fmt, size_t n, size_t k, size_t bucket,
                           int row_invariant, jv_plan plan);
void jv_tuner_insert_grouped(jv_tuner *t, uint32_t fmt, size_t n, size_t k, size_t experts,
                             size_t bucket, uint32_t bm, uint32_t bn);
/* Tuner::dense (tune.rs:162-174) and Tuner::grouped (tune.rs:177-190). */
jv_plan jv_tuner_dense(const jv_tuner *t, const jv_qmatrix *w, size_t m, int row_invariant);
jv_status jv_tuner_grouped(const jv_tuner *t, const jv_qmatrix *w, size_t rows, uint32_t *bm,
                           uint32_t *bn);
/* Measures the candidate plans for matrices `ws` of one shape at m = bucket rows (tune_dense,
 * tune.rs:229-268); x, out are scratch of at least m*k and m*n values. *added = 1 when a plan
 * was stored. */
jv_status jv_tuner_tune_dense(jv_tuner *t, const jv_qmatrix *const *ws, size_t nws, size_t m,
                              int row_invariant, const void *x, jv_act act, size_t x_len,
                              void *out, size_t out_len, jv_scratch *scratch, int *added);
/* Measures the grouped tiles for `rows` tokens routed to top_k experts each (tune_grouped,
 * tune.rs:270-343); route_ids, sorted, offsets, jobs are device scratch (route_capacity ids). */
jv_status jv_tuner_tune_grouped(jv_tuner *t, const jv_qmatrix *const *ws, size_t nws, size_t rows,
                                size_t top_k, const void *x, jv_act act, size_t x_len, void *out,
                                size_t out_len, uint32_t *route_ids, size_t route_capacity,
                                uint32_t *sorted, uint32_t *offsets, uint32_t *jobs,
                                size_t jobs_len, jv_scratch *scratch, int *added);
/* Writes the table (Tuner::save, tune.rs:413-444): the profile line, then sorted entries. */
jv_status jv_tuner_save(const jv_tuner *t);

/* ---------------------------------------------------------------------------------------------
 * GGUF v2/v3 reader (Gguf, crates/jevons-formats/src/gguf.rs:163-372): validated metadata,
 * tensor directory (absolute offsets, byte sizes of the block-encoded types) and bounded reads;
 * errors carry the reference's messages ("Invalid GGUF file: ...", "Missing tensor ...").
 * ------------------------------------------------------------------------------------------ */
typedef struct jv_gguf jv_gguf;
jv_status jv_gguf_open(const char *path, jv_gguf **out);  /* Gguf::open (gguf.rs:234-321) */
void jv_gguf_close(jv_gguf *g);
size_t jv_gguf_tensor_count(const jv_gguf *g);
/* TensorInfo (gguf.rs:146-155): dims in GGML order (dims[0] = row length), unused dims = 1;
 * bytes = 0 for types without a block size. */
jv_status jv_gguf_tensor_info(const jv_gguf *g, size_t index, const char **name,
                              uint32_t *ggml_type, uint32_t *n_dims, uint64_t dims[4],
                              uint64_t *offset, uint64_t *bytes);
jv_status jv_gguf_find(const jv_gguf *g, const char *name, size_t *index);  /* Gguf::tensor */
jv_status jv_gguf_u64(const jv_gguf *g, const char *key, uint64_t *out);    /* Gguf::u64 */
jv_status jv_gguf_f32(const jv_gguf *g, const char *key, float *out);       /* Gguf::f32 */
jv_status jv_gguf_str(const jv_gguf *g, const char *key, const char **out);
/* Gguf::read / read_range (gguf.rs:338-362): bytes [start, start + len) of a tensor of a
 * decodable type into host memory. */
jv_status jv_gguf_read(const jv_gguf *g, size_t index, uint64_t start, uint64_t len, void *dst);
/* Reads a [k, n] or [k, n, experts] tensor and uploads it (QMatrix::upload, gemm.rs:822-841;
 * the loader step of model.rs:302-351). */
jv_status jv_gguf_upload(jv_ctx *ctx, const jv_gguf *g, const char *name, jv_qmatrix **out);

/* Message of the last failed call on this thread ("" if none). */
const char *jv_last_error(void);

#ifdef __cplusplus
}
#endif
#endif

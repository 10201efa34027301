/*
 * jv_oracle.h — CPU oracle for the quantized GGML matmul path (TEST INFRASTRUCTURE ONLY).
 *
 * A plain-C restatement of the reference's CPU block decode, packing, type table, f64 matmul
 * and greedy argmax. Only tests/, the smoke check and the CPU-baseline leg of bench.py load
 * this library, and only as the checker or the timed CPU baseline; the product path never
 * calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference
 * repository root).
 */
#ifndef JV_ORACLE_H
#define JV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (crates/jevons-formats/src/gguf.rs:120-131). */
enum { JVO_F32 = 0, JVO_F16 = 1, JVO_Q5_0 = 6, JVO_Q8_0 = 8, JVO_Q4K = 12, JVO_Q6K = 14 };

/* (elements per block, bytes per block) of a GGML type id; returns 0 for unsupported ids
 * (gguf.rs:134-144). */
int jvo_type_block(uint32_t type_id, uint32_t *elems, uint32_t *bytes);

/* IEEE binary16 <-> binary32 (the `half` 2.7.1 conversions used by quant.rs:9-11 and the
 * test fixtures' `f16::from_f32`). f32->f16 rounds to nearest even. */
float jvo_f16_to_f32(uint16_t h);
uint16_t jvo_f32_to_f16(float f);
/* bfloat16 -> f32 (exact) and f32 -> bf16 (round to nearest even). */
float jvo_bf16_to_f32(uint16_t h);
uint16_t jvo_f32_to_bf16(float f);

/* Q4_K 6-bit (scale, min) pair j of the 12 packed scale bytes (quant.rs:14-23). */
void jvo_q4k_scale_min(int j, const uint8_t *q, uint8_t *scale, uint8_t *min);

/* One-block decoders (quant.rs:25-80). */
void jvo_dequant_q4k(const uint8_t *block, float *out);
void jvo_dequant_q6k(const uint8_t *block, float *out);
void jvo_dequant_q5_0(const uint8_t *block, float *out);
void jvo_dequant_q8_0(const uint8_t *block, float *out);

/* Whole-tensor decode with the reference's size checks (quant.rs:83-101).
 * Returns 0 on success, 1 "unsupported tensor type", 2 "dequantization size mismatch". */
int jvo_dequantize(uint32_t type_id, const uint8_t *bytes, size_t nbytes, float *out, size_t nout);

/* Words per block of each packed region (q, h, s, d) (quant.rs:127-135). */
void jvo_packed_words(uint32_t type_id, size_t *q, size_t *h, size_t *s, size_t *d);

/* The reference's structure-of-arrays repack (quant.rs:156-193). Regions must be sized by
 * jvo_packed_words * blocks. Returns 0, 1 "unsupported tensor type", 2 "not a whole number of
 * blocks", 3 "no GPU block layout". */
int jvo_pack(uint32_t type_id, const uint8_t *bytes, size_t nbytes, uint32_t *q, uint32_t *h,
             uint32_t *s, float *d);

/* f64 product out[r, c] = sum_k x[r, k] * w[c, k] (crates/jevons-gemma4-diffusion/src/gpu/
 * tests.rs:445-451). x is [m, k] f32, w is [n, k] f32, out is [m, n] f64. OpenMP over rows. */
void jvo_matmul_f64(const float *x, size_t m, size_t k, const float *w, size_t n, double *out);

/* Greedy argmax of one row: first maximum wins (strict `>` fold), non-finite or empty is an
 * error (crates/jevons-core/src/model.rs:207-219). Returns 0 ok, 1 error. prob = 1/sum exp. */
int jvo_greedy(const float *row, size_t n, int32_t *index, double *prob);

/* xorshift64 fixture generator of the reference GPU tests (gpu/tests.rs:11-23):
 * state ^= state<<13; ^= >>7; ^= <<17; value = (state>>40)/2^24*2-1 in [-1, 1). */
float jvo_rng_next(uint64_t *state);

/* Reference test recipes built on jvo_rng_next:
 * Q8_0 weights of gpu/tests.rs:431-436 (d = f16(0.01+|u|*0.02), q = (u*100) as i8);
 * Q6_K table of gpu/tests.rs:546-554 (ql/qh = (|u|*255) as u8, sc = (u*100) as i8,
 * d = f16(0.001+|u|*0.01)). Output sized blocks*34 / blocks*210 bytes. */
void jvo_recipe_q8_0(uint64_t *state, size_t blocks, uint8_t *out);
void jvo_recipe_q6k(uint64_t *state, size_t blocks, uint8_t *out);
/* rng.vec(n, scale) then h16 (round through f16), as f32 values (gpu/tests.rs:20-27). */
void jvo_recipe_h16_vec(uint64_t *state, size_t n, float scale, float *out);

/* CPU baseline: the reference CPU path (dequantize, quant.rs:83-101, then a row-major f32
 * accumulate x . W^T). threads <= 0 uses every OpenMP thread. wdec is caller scratch of
 * n*k floats; when decode == 0 it must already hold the decoded weights. Returns the status of
 * the decode. */
int jvo_cpu_dequant_matmul(uint32_t type_id, const uint8_t *bytes, size_t n, size_t k,
                           const float *x, size_t m, float *out, float *wdec, int decode,
                           int threads);
int jvo_omp_max_threads(void);

/* ops::group (gpu/ops.rs:522-587): expert grouping of routed assignments (ids >= experts are
 * not routed). Returns the job count. */
int jvo_group_routes(const uint32_t *ids, size_t assignments, size_t experts, size_t bm,
                     uint32_t *sorted, uint32_t *offsets, uint32_t *jobs);

#ifdef __cplusplus
}
#endif
#endif

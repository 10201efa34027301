// Launch parameters shared by the host library and the gfx950 kernels (passed by value).
#ifndef JV_QMM_PARAMS_H
#define JV_QMM_PARAMS_H

#include <stdint.h>

// Product out[m, n] = sum_k x[m, k] * W[n, k]. Weight regions follow the device layout of the
// weight format (see the format decoders in kernels/qmm.hip).
struct QmmParams {
    const void *x;       // activations [M][ldx], element type `act`
    void *out;           // [M][ldo] of `out_type`, or FP32 split partials when splits > 1
    const uint8_t *wq;   // quant region
    const uint8_t *wh;   // high-bit region (Q5_0)
    const uint8_t *wd;   // FP16 block scales (Q6_K, Q8_0, Q5_0)
    int32_t M, N, K;     // N = weight rows, K = reduction length
    int32_t ldx, ldo;    // row strides in elements
    int32_t act;         // 0 f16, 1 bf16, 2 f32
    int32_t out_type;    // 0 f32, 1 bf16 (ignored for split partials, which are f32)
    int32_t kc;          // K staged in LDS per chunk (multiple of the format's K unit)
    int32_t splits;      // grid z; slice z covers units [z*U/splits, (z+1)*U/splits)
    int64_t split_stride;  // elements between partial planes
    // Expert-grouped mode (grid y = job; gemm.rs:9-11): job j covers sorted positions
    // [jobs[2j+2], min(+rows_cap, offsets[e+1])) of expert e = jobs[2j+1]; position s reads
    // input row ids[s] / in_div and writes output row ids[s]; weight rows start at e * N.
    const uint32_t *ids, *offsets, *jobs;
    int32_t grouped, in_div, rows_cap;
    // Split-K small-row kernels: FP32 slice partials [slices][M][N] and one arrival counter per
    // 16-row tile (kept at a multiple of 16 between launches).
    float *part;
    uint32_t *counters;
    // Tiled kernels: per input row, the factor that undoes the row's range scale (multiplied
    // into its outputs); null for none. The activations were then prescaled FP16 rows.
    const float *rscale;
    // Greedy epilogue (persistent small-row kernels): as GemmParams' below.
    float cap;
    uint64_t *amax_key;
    uint32_t *amax_bad;
};

// Decode probe: rows [row0, row0 + rows) of a weight matrix into [rows][K].
struct DequantParams {
    const uint8_t *wq;
    const uint8_t *wh;
    const uint8_t *wd;
    void *out;
    int32_t K;
    int32_t row0, rows;
    int32_t f16_out;     // 0: FP32 values, 1: FP16 tile values
};

// Activation rows -> FP16 MFMA A fragments of 1 KB: fragment (mt * U + u) * 8 + s (U = K / 256)
// holds, for lane 16g + r, x[16 mt + r][256 u + 32 s + 8 g + e], e < 8; rows >= M (and a job's
// rows past its count) are not written, and no product stores their outputs.
// Rows of BF16 or FP32 values above 16384 are divided by a power-of-two range factor first;
// rscale[R] gets packed row R's factor, for the product to undo. With `rowmajor` (BF16 and
// FP32 only, never grouped) the output is FP16 rows [M][K] and rscale per row.
struct PackXParams {
    const void *x;       // [M][ldx] of `act`
    uint16_t *out;       // FP16 bits, mtiles * (K / 32) fragments of 512 elements (or [M][K])
    float *rscale;       // [mtiles * 16] (or [M])
    int32_t M, K, ldx, act;
    int32_t mtiles;      // 16-row tiles packed (M rounded up to the product's row tile)
    int32_t rowmajor;
    int32_t rpw;         // BF16 / FP32: rows per workgroup (1, 2 or 4)
    // Expert-grouped mode: m-tiles [j rows_cap / 16, (j + 1) rows_cap / 16) hold job j's rows,
    // input rows ids[s] / in_div for sorted positions s of the job (QmmParams' job format).
    const uint32_t *ids, *offsets, *jobs;
    int32_t grouped, in_div, rows_cap;
};

// Tiled product over packed activation fragments (jv_pack_x output).
struct GemmParams {
    const uint16_t *xa;  // packed activations
    const uint8_t *wq;   // weight regions of the format's device layout
    const uint8_t *wh;
    const uint8_t *wd;
    void *out;           // [M][ldo] of `out_type`
    const float *rscale; // per packed row, the factor undoing its range scale (jv_pack_x)
    int32_t M, N, K, ldo, out_type;
    // Expert-grouped mode (grid y = job): the job's rows come packed per job, its weight rows
    // start at expert * N, and its output rows are ids[start + r] (QmmParams' job format).
    const uint32_t *ids, *offsets, *jobs;
    int32_t grouped, rows_cap;
    // Split-K (ungrouped): grid z = slice; slice z covers the format's K units
    // [z U / splits, (z + 1) U / splits), each a whole number of 256-element blocks, and writes
    // FP32 partials to part + z * split_stride ([M][ldo]), summed by jv_reduce_splits.
    float *part;
    int64_t split_stride;
    int32_t splits;
    // Greedy epilogue (ungrouped, whole K, FP32 outputs), in the kernels built with it: every
    // output value is soft-capped, cap tanh(v / cap), when cap > 0, then stored, and each
    // workgroup folds, per output row it covers, the largest of its columns' values and that
    // value's first column into amax_key[row] (an atomic maximum of the ordered value bits over
    // the inverted column) or sets amax_bad[row] when one of its values is not finite; both start
    // at zero, and jv_greedy_finish, launched after the product, turns them into the rows'
    // columns and zeroes them again.
    float cap;
    uint64_t *amax_key;
    uint32_t *amax_bad;
};

// GGML blocks (device copy of the upload) -> device layout.
struct RepackParams {
    const uint8_t *raw;
    uint8_t *wq;
    uint8_t *wh;
    uint8_t *wd;
    int64_t chunks;      // work items (format-specific unit of the repack)
};


// Candidate logits (pick_logits): out[p] = cap tanh(x[row] . E[token] / cap), pair p = (row, token).
struct PickParams {
    const void *x;         // activations [x_rows][d], element type `act`
    const uint32_t *pairs; // (row, token) pairs
    const uint8_t *wq, *wh, *wd;  // the table's device regions
    float *out;            // [count]
    int32_t d, act, count, x_rows, n;
    float cap;
};

#endif

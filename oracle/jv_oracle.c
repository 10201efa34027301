/*
 * jv_oracle.c — CPU oracle for the quantized GGML matmul path (TEST INFRASTRUCTURE ONLY).
 *
 * Restates, in plain C, the reference's CPU block decode (crates/jevons-formats/src/quant.rs),
 * its GGML type table (crates/jevons-formats/src/gguf.rs), the f64 product its GPU tests
 * compare against (crates/jevons-gemma4-diffusion/src/gpu/tests.rs) and its greedy argmax
 * (crates/jevons-core/src/model.rs). Only tests/, the smoke check and bench.py's CPU-baseline
 * leg load this library; the product path never does.
 *
 * The f16 conversions are written from the IEEE 754 binary16 definition; the reference gets
 * them from the `half` 2.7.1 crate (Cargo.lock), whose conversions are exact (f16->f32) and
 * round to nearest even (f32->f16), which is all the definition allows.
 */
#include "jv_oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* gguf.rs:120-144: TensorType::from_id and TensorType::block. */
int jvo_type_block(uint32_t type_id, uint32_t *elems, uint32_t *bytes) {
    uint32_t e = 0, b = 0;
    switch (type_id) {
    case JVO_F32: e = 1; b = 4; break;
    case JVO_F16: e = 1; b = 2; break;
    case JVO_Q5_0: e = 32; b = 22; break;
    case JVO_Q8_0: e = 32; b = 34; break;
    case JVO_Q4K: e = 256; b = 144; break;
    case JVO_Q6K: e = 256; b = 210; break;
    default: return 0;
    }
    if (elems) *elems = e;
    if (bytes) *bytes = b;
    return 1;
}

/* quant.rs:9-11 (`half(bytes)` = f16::from_le_bytes(..).to_f32()). */
float jvo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        float v = (float)man * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 31) {
        /* infinity, or NaN with its payload (quiet bit set) */
        return bits_f32(sign | 0x7f800000u | (man ? (0x00400000u | (man << 13)) : 0u));
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* `f16::from_f32` (round to nearest, ties to even). */
uint16_t jvo_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    int32_t e16 = (int32_t)exp - 112; /* biased binary16 exponent */
    if (e16 >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e16 <= 0) {
        /* result is subnormal (or zero): value / 2^-24 = (1.man) * 2^(exp - 126) */
        if (e16 < -10) return (uint16_t)sign;
        uint32_t full = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e16);
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e16 << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carry may reach infinity */
    return (uint16_t)(sign | q);
}

float jvo_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t jvo_f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

static float half_at(const uint8_t *p) { return jvo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* quant.rs:14-23 */
void jvo_q4k_scale_min(int j, const uint8_t *q, uint8_t *scale, uint8_t *min) {
    if (j < 4) {
        *scale = q[j] & 63;
        *min = q[j + 4] & 63;
    } else {
        *scale = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *min = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant.rs:25-41: w[64p+l] = d*s_{2p}*(qs[32p+l]&15) - dmin*m_{2p}, high nibble -> +32. */
void jvo_dequant_q4k(const uint8_t *block, float *out) {
    float d = half_at(block), dmin = half_at(block + 2);
    const uint8_t *scales = block + 4, *qs = block + 16;
    for (int pair = 0; pair < 4; pair++) {
        uint8_t s0, m0, s1, m1;
        jvo_q4k_scale_min(2 * pair, scales, &s0, &m0);
        jvo_q4k_scale_min(2 * pair + 1, scales, &s1, &m1);
        float d0 = d * (float)s0, n0 = dmin * (float)m0;
        float d1 = d * (float)s1, n1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[pair * 32 + l];
            /* built with -ffp-contract=off: product, then one rounded subtraction, as Rust */
            out[pair * 64 + l] = d0 * (float)(q & 15) - n0;
            out[pair * 64 + 32 + l] = d1 * (float)(q >> 4) - n1;
        }
    }
}

/* quant.rs:43-61: ql 128 B, qh 64 B, sc 16 x i8, f16 d; two 128-element halves. */
void jvo_dequant_q6k(const uint8_t *block, float *out) {
    float d = half_at(block + 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = block + 64 * n, *qh = block + 128 + 32 * n;
        const int8_t *sc = (const int8_t *)(block + 192 + 8 * n);
        float *o = out + 128 * n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = ((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
            int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            /* Rust evaluates d * f32(sc) first, then * q (left to right) */
            float s1 = d * (float)sc[is], s2 = d * (float)sc[is + 2];
            float s3 = d * (float)sc[is + 4], s4 = d * (float)sc[is + 6];
            o[l] = s1 * (float)q1;
            o[l + 32] = s2 * (float)q2;
            o[l + 64] = s3 * (float)q3;
            o[l + 96] = s4 * (float)q4;
        }
    }
}

/* quant.rs:63-73 */
void jvo_dequant_q5_0(const uint8_t *block, float *out) {
    float d = half_at(block);
    uint32_t qh = (uint32_t)block[2] | ((uint32_t)block[3] << 8) | ((uint32_t)block[4] << 16) |
                  ((uint32_t)block[5] << 24);
    const uint8_t *qs = block + 6;
    for (int j = 0; j < 16; j++) {
        uint32_t h0 = ((qh >> j) << 4) & 0x10u;
        uint32_t h1 = (qh >> (j + 12)) & 0x10u;
        out[j] = d * (float)((int32_t)((qs[j] & 15u) | h0) - 16);
        out[j + 16] = d * (float)((int32_t)((uint32_t)(qs[j] >> 4) | h1) - 16);
    }
}

/* quant.rs:75-80 */
void jvo_dequant_q8_0(const uint8_t *block, float *out) {
    float d = half_at(block);
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)block[2 + i];
}

/* quant.rs:83-101 */
int jvo_dequantize(uint32_t type_id, const uint8_t *bytes, size_t nbytes, float *out, size_t nout) {
    uint32_t block, size;
    if (!jvo_type_block(type_id, &block, &size)) return 1;
    if (nbytes % size != 0 || nout != nbytes / size * block) return 2;
    size_t blocks = nbytes / size;
#pragma omp parallel for schedule(static) if (blocks > 4096)
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t *src = bytes + b * size;
        float *dst = out + b * block;
        switch (type_id) {
        case JVO_F32: memcpy(dst, src, 4); break;
        case JVO_F16: dst[0] = half_at(src); break;
        case JVO_Q4K: jvo_dequant_q4k(src, dst); break;
        case JVO_Q6K: jvo_dequant_q6k(src, dst); break;
        case JVO_Q5_0: jvo_dequant_q5_0(src, dst); break;
        case JVO_Q8_0: jvo_dequant_q8_0(src, dst); break;
        }
    }
    return 0;
}

/* quant.rs:127-135 */
void jvo_packed_words(uint32_t type_id, size_t *q, size_t *h, size_t *s, size_t *d) {
    size_t w[4] = {0, 0, 0, 0};
    switch (type_id) {
    case JVO_Q4K: w[0] = 36; break;
    case JVO_Q6K: w[0] = 32; w[1] = 16; w[2] = 4; w[3] = 1; break;
    case JVO_Q5_0: w[0] = 4; w[1] = 1; w[3] = 1; break;
    case JVO_Q8_0: w[0] = 8; w[3] = 1; break;
    }
    *q = w[0]; *h = w[1]; *s = w[2]; *d = w[3];
}

static void le_words(const uint8_t *b, size_t nbytes, uint32_t *out) {
    for (size_t i = 0; i + 4 <= nbytes; i += 4)
        out[i / 4] = (uint32_t)b[i] | ((uint32_t)b[i + 1] << 8) | ((uint32_t)b[i + 2] << 16) |
                     ((uint32_t)b[i + 3] << 24);
}

/* quant.rs:156-193 */
int jvo_pack(uint32_t type_id, const uint8_t *bytes, size_t nbytes, uint32_t *q, uint32_t *h,
             uint32_t *s, float *d) {
    uint32_t block, size;
    if (!jvo_type_block(type_id, &block, &size)) return 1;
    if (nbytes % size != 0) return 2;
    size_t blocks = nbytes / size;
    switch (type_id) {
    case JVO_Q4K: le_words(bytes, nbytes, q); break;
    case JVO_Q6K:
        for (size_t i = 0; i < blocks; i++) {
            const uint8_t *b = bytes + i * size;
            le_words(b, 128, q + 32 * i);
            le_words(b + 128, 64, h + 16 * i);
            le_words(b + 192, 16, s + 4 * i);
            d[i] = half_at(b + 208);
        }
        break;
    case JVO_Q5_0:
        for (size_t i = 0; i < blocks; i++) {
            const uint8_t *b = bytes + i * size;
            d[i] = half_at(b);
            le_words(b + 2, 4, h + i);
            le_words(b + 6, 16, q + 4 * i);
        }
        break;
    case JVO_Q8_0:
        for (size_t i = 0; i < blocks; i++) {
            const uint8_t *b = bytes + i * size;
            d[i] = half_at(b);
            le_words(b + 2, 32, q + 8 * i);
        }
        break;
    default: return 3;
    }
    return 0;
}

/* gpu/tests.rs:445-451 (f64 sum over k of f64(x) * f64(w)). */
void jvo_matmul_f64(const float *x, size_t m, size_t k, const float *w, size_t n, double *out) {
    long long total = (long long)(m * n);
#pragma omp parallel for schedule(static) if (total * (long long)k > 1000000)
    for (long long i = 0; i < total; i++) {
        size_t r = (size_t)i / n, c = (size_t)i % n;
        const float *xr = x + r * k, *wc = w + c * k;
        double acc = 0.0;
        for (size_t j = 0; j < k; j++) acc += (double)xr[j] * (double)wc[j];
        out[i] = acc;
    }
}

/* crates/jevons-core/src/model.rs:207-219 */
int jvo_greedy(const float *row, size_t n, int32_t *index, double *prob) {
    if (n == 0) return 1;
    for (size_t i = 0; i < n; i++)
        if (!isfinite(row[i])) return 1;
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (row[i] > row[best]) best = i;
    double max = (double)row[best], z = 0.0;
    for (size_t i = 0; i < n; i++) z += exp((double)row[i] - max);
    *index = (int32_t)best;
    if (prob) *prob = 1.0 / z;
    return 0;
}

/* ops::group (crates/jevons-gemma4-diffusion/src/gpu/ops.rs:522-587): assignments sorted by
 * expert, stable within an expert (sorted[...] = assignment index); offsets[e] = first sorted
 * position of expert e, offsets[experts] = assignments; jobs[0] = job count, then one
 * (expert, start) pair per bm-row tile of each expert, experts in order. Ids >= experts match no
 * expert and are not routed, as in the reference kernel. Returns the job count. */
int jvo_group_routes(const uint32_t *ids, size_t assignments, size_t experts, size_t bm,
                     uint32_t *sorted, uint32_t *offsets, uint32_t *jobs) {
    uint32_t acc = 0, jacc = 0;
    for (size_t e = 0; e < experts; e++) {
        uint32_t count = 0;
        for (size_t a = 0; a < assignments; a++) count += ids[a] == e;
        offsets[e] = acc;
        uint32_t next = acc;
        for (size_t a = 0; a < assignments; a++)
            if (ids[a] == e) sorted[next++] = (uint32_t)a;
        const uint32_t tiles = (uint32_t)((count + bm - 1) / bm);
        for (uint32_t t = 0; t < tiles; t++) {
            jobs[1 + 2 * (jacc + t)] = (uint32_t)e;
            jobs[2 + 2 * (jacc + t)] = acc + t * (uint32_t)bm;
        }
        acc += count;
        jacc += tiles;
    }
    offsets[experts] = acc;
    jobs[0] = jacc;
    return (int)jacc;
}

/* gpu/tests.rs:11-23 */
float jvo_rng_next(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (float)(x >> 40) / (float)(1ull << 24) * 2.0f - 1.0f;
}

/* Rust `f as i8` / `f as u8`: truncate toward zero, saturate at the type's bounds. */
static int8_t as_i8(float f) {
    if (f != f) return 0;
    if (f >= 127.0f) return 127;
    if (f <= -128.0f) return -128;
    return (int8_t)f;
}

static uint8_t as_u8(float f) {
    if (f != f || f <= 0.0f) return 0;
    if (f >= 255.0f) return 255;
    return (uint8_t)f;
}

/* gpu/tests.rs:431-436 */
void jvo_recipe_q8_0(uint64_t *state, size_t blocks, uint8_t *out) {
    for (size_t b = 0; b < blocks; b++) {
        uint8_t *o = out + 34 * b;
        uint16_t d = jvo_f32_to_f16(0.01f + fabsf(jvo_rng_next(state)) * 0.02f);
        o[0] = (uint8_t)(d & 0xff);
        o[1] = (uint8_t)(d >> 8);
        for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)as_i8(jvo_rng_next(state) * 100.0f);
    }
}

/* gpu/tests.rs:546-554 */
void jvo_recipe_q6k(uint64_t *state, size_t blocks, uint8_t *out) {
    for (size_t b = 0; b < blocks; b++) {
        uint8_t *o = out + 210 * b;
        for (int i = 0; i < 192; i++) o[i] = as_u8(fabsf(jvo_rng_next(state)) * 255.0f);
        for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t)as_i8(jvo_rng_next(state) * 100.0f);
        uint16_t d = jvo_f32_to_f16(0.001f + fabsf(jvo_rng_next(state)) * 0.01f);
        o[208] = (uint8_t)(d & 0xff);
        o[209] = (uint8_t)(d >> 8);
    }
}

/* gpu/tests.rs:20-27 (rng.vec then h16) */
void jvo_recipe_h16_vec(uint64_t *state, size_t n, float scale, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = jvo_f16_to_f32(jvo_f32_to_f16(jvo_rng_next(state) * scale));
}

int jvo_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* CPU baseline: quant.rs:83-101 decode, then a row-major f32-accumulate x . W^T. */
int jvo_cpu_dequant_matmul(uint32_t type_id, const uint8_t *bytes, size_t n, size_t k,
                           const float *x, size_t m, float *out, float *wdec, int decode,
                           int threads) {
    uint32_t block, size;
    if (!jvo_type_block(type_id, &block, &size)) return 1;
    if (k % block != 0) return 2;
    size_t row_bytes = k / block * size;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#else
    int nt = 1;
    (void)threads;
#endif
    int status = 0;
#pragma omp parallel num_threads(nt)
    {
        if (decode) {
#pragma omp for schedule(static)
            for (long long c = 0; c < (long long)n; c++) {
                const uint8_t *src = bytes + (size_t)c * row_bytes;
                float *dst = wdec + (size_t)c * k;
                for (size_t b = 0; b < k / block; b++) {
                    const uint8_t *blk = src + b * size;
                    float *o = dst + b * block;
                    switch (type_id) {
                    case JVO_F32: memcpy(o, blk, 4); break;
                    case JVO_F16: o[0] = half_at(blk); break;
                    case JVO_Q4K: jvo_dequant_q4k(blk, o); break;
                    case JVO_Q6K: jvo_dequant_q6k(blk, o); break;
                    case JVO_Q5_0: jvo_dequant_q5_0(blk, o); break;
                    case JVO_Q8_0: jvo_dequant_q8_0(blk, o); break;
                    }
                }
            }
        }
#pragma omp for schedule(static)
        for (long long c = 0; c < (long long)n; c++) {
            const float *wc = wdec + (size_t)c * k;
            for (size_t r = 0; r < m; r++) {
                const float *xr = x + r * k;
                float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
                for (size_t j = 0; j < k; j++) acc += xr[j] * wc[j];
                out[r * n + (size_t)c] = acc;
            }
        }
    }
    return status;
}

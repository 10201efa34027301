// gfx950 (CDNA4, wave64) kernels for products with GGML-quantized weights.
//
// out[m, n] = sum_k x[m, k] * W[n, k], FP32 accumulation on MFMA 16x16x32 f16.
//
// Work decomposition (one kernel for every plan): a workgroup of 4 waves owns the output tile
// rows [m0, m0 + 16*MT) x columns [n0, n0 + 4*16*NT). Each wave owns 16*NT weight rows and all
// 16*MT activation rows of the tile, so every weight is fetched from HBM and decoded exactly
// once per workgroup, straight into MFMA B-operand registers; no LDS round trip for weights.
// The activation tile is staged once per K chunk in LDS as FP16 and shared by the 4 waves.
//
// Lane roles inside a wave (lane = 16*g + r, r = lane % 16, g = lane / 16):
//   A operand (activations): row r of the 16-row m-subtile, 8 consecutive k of group g;
//   B operand (weights):     weight row r of the 16-row n-subtile, the same 8 k;
//   accumulator:             column r, rows 4*g .. 4*g+3 (MFMA 16x16 f32 layout).
// Which 8 k a lane group holds at each 32-k step is chosen per format so a lane's weight bytes
// for a whole K unit are one or a few contiguous 16-byte loads; the activation fragment is
// read at the matching k offset (F::kidx), so the contraction is the same sum in any order.
//
// Weights are decoded to FP32 exactly as the reference's CPU decode computes them
// (crates/jevons-formats/src/quant.rs:25-80: exact products, one rounding where quant.rs has
// one) and rounded to nearest even into FP16 for the MFMA, which is the reference's on-chip
// tile format (crates/jevons-kernels/src/gemm.rs:131-284).
//
// Every output element is accumulated by the same sequence of MFMA steps over K whatever the
// plan's row and column tiles are, so plans without split-K give bitwise-identical rows.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../qmm_params.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Plain vector (not HIP's uint4 struct): arrays of it stay in registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kLdsPad = 8;  // FP16 elements of padding per staged activation row (16 bytes)

// Workgroup barrier ordering LDS only. __syncthreads() fences every address space, which on
// gfx950 waits for all outstanding global loads (vmcnt(0)) and so drains the weight prefetch
// queued ahead of the barrier; this one waits for LDS traffic (lgkmcnt(0)) alone.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}

__device__ __forceinline__ float bf2f(uint32_t bits16) {
    return __builtin_bit_cast(float, (bits16 & 0xffffu) << 16);
}

__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (x >> 16) | 0x40u;
    return (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
}

// FP32 -> FP16, round to nearest even, of a value already rounded to FP32. The empty asm keeps
// the compiler from fusing a preceding fma into v_fma_mix{lo,hi}_f16, which rounds the exact
// product-sum to FP16 once; quant.rs rounds to FP32 first, and the two differ on ties. It is not
// volatile: a volatile asm would also end the instruction scheduler's region at every element.
__device__ __forceinline__ _Float16 f32_to_f16(float v) {
    asm("" : "+v"(v));
    return (_Float16)v;
}

typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
// Bytes (0, 2) (SEL 0x05020500) or (1, 3) (SEL 0x05030501) of w as two FP16 integers, each
// byte b minus the bias whose -(1024 + bias) pair is nbias2: 0x64 above a byte makes the FP16
// value 1024 + b, and the packed FP16 addition of these integers is exact.
template <uint32_t SEL>
__device__ __forceinline__ h16x2 bytes_f16_minus(uint32_t w, uint32_t nbias2) {
    return __builtin_bit_cast(h16x2, __builtin_amdgcn_perm(0x64646464u, w, SEL)) +
           __builtin_bit_cast(h16x2, nbias2);
}
// -0.0f in a scalar register the compiler cannot see through: fma(h, s, -0) is bitwise s * h
// (x + -0 is x for every x, +-0 included), and with an opaque addend the compiler keeps it as
// one v_fma_mix_f32 (FP16 operand converted inside) instead of folding it to a conversion and
// a v_mul_f32.
__device__ __forceinline__ float opaque_neg_zero() {
    uint32_t z;
    asm("" : "=s"(z) : "0"(0x80000000u));
    return __builtin_bit_cast(float, z);
}

__device__ __forceinline__ f16x8 pack8(const float v[8]) {
    f16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = f32_to_f16(v[e]);
    return r;
}

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *(const uint4 *)p; }

// ---------------------------------------------------------------------------------------------
// Format decoders. Each provides:
//   KU          K elements per unit (one load group per lane)
//   Raw         the lane's raw bytes of one unit of one weight row
//   load()      fetch them (16-byte loads)
//   Prep/prep() per-unit scales the lane needs
//   kidx(s, g)  k offset inside the unit of lane group g's 8 elements at 32-k step s
//   frag_f32()  those 8 weights, decoded exactly as quant.rs does
// ---------------------------------------------------------------------------------------------

// Q4_K, device layout: GGUF blocks (f16 d, f16 dmin, 12 scale bytes, 128 quant bytes) regrouped
// per 16-row tile and block into 2304 contiguous bytes, tile-major then block:
//   [0, 1024)     lane 16g + r: quant bytes 8g..8g+7 of pairs 0 and 1 of row r's block
//   [1024, 2048)  lane 16g + r: the same bytes of pairs 2 and 3
//   [2048, 2304)  the 16 rows' 16-byte heads (d, dmin, scales)
// where pair p is quant bytes 32p..32p+31 and each 4-byte group is stored in the order
// {0, 2, 1, 3}. Each 16-byte load of a wave reads 1 KB (or the 256-byte heads) contiguously.
// Lane group g thus holds elements 32j + 8g + e of every sub-block j (low nibbles of pair j/2
// for even j, high nibbles for odd j; quant.rs:25-41), and the {0, 2, 1, 3} order makes
// (w & 0x000f000f) hold the nibbles of elements e, e+1 in its two 16-bit halves.
__device__ __forceinline__ uint32_t q4k_nib(uint32_t w, int e, int h) {
    // element e (0..3) of a stored word, nibble h: byte position {0, 2, 1, 3}[e]
    const int pos = (e == 1) ? 2 : (e == 2 ? 1 : e);
    return (w >> (8 * pos + 4 * h)) & 15u;
}

// (scale, min) of Q4_K sub-block j from the 12 scale bytes held in hd.y..hd.w (quant.rs:14-23)
__device__ __forceinline__ void q4k_scale_min_dev(const uint4 &hd, int j, uint32_t &sc, uint32_t &mn) {
    const int sh = 8 * (j & 3);
    const uint32_t a = hd.y >> sh, b = hd.z >> sh, c = hd.w >> sh;
    if (j < 4) {
        sc = a & 63u;
        mn = b & 63u;
    } else {
        sc = (c & 15u) | ((a >> 2) & 48u);
        mn = ((c >> 4) & 15u) | ((b >> 2) & 48u);
    }
}

struct FQ4K {
    static constexpr int KU = 256;
    struct Raw {
        uint4 hd, q0, q1;
    };
    struct Prep {
        float dd[8], mm[8];
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *,
                                int K, int row, int u, int g) {
        const int rr = row & 15;
        const uint8_t *tb = wq + ((size_t)(row >> 4) * (size_t)(K / 256) + (size_t)u) * 2304u;
        r.q0 = ld16(tb + (16 * g + rr) * 16);
        r.q1 = ld16(tb + 1024 + (16 * g + rr) * 16);
        r.hd = ld16(tb + 2048 + rr * 16);
    }
    __device__ static void prep(const Raw &r, Prep &p, int) {
        const float d = h2f(r.hd.x), dmin = h2f(r.hd.x >> 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, mn;
            q4k_scale_min_dev(r.hd, j, sc, mn);
            p.dd[j] = d * (float)sc;     // exact: 11 x 6 significant bits
            p.mm[j] = dmin * (float)mn;  // exact
        }
    }
    __device__ static int kidx(int s, int g) { return 32 * s + 8 * g; }
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int, float v[8]) {
        const int pr = s >> 1, h = s & 1;
        const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // d*s*q is exact, so one fused rounding equals quant.rs's product-then-subtract.
            v[e] = __builtin_fmaf((float)q4k_nib(w[2 * pr + (e >> 2)], e & 3, h), p.dd[s], -p.mm[s]);
        }
    }
};

// Q6_K, device layout: 16-row tiles, per 256 k 3360 bytes. Lane 16g + r owns 48 bytes of row r,
// in three 16-byte pieces at [0, 1024), [1024, 2048), [2048, 3072) (piece i at 1024 i + 16 lane):
// ql(hf, i2) = ql[64hf + 32i2 + 8g, +8) for (hf, i2) = (0,0), (0,1), (1,0), (1,1), then
// qh(hf) = qh[32hf + 8g, +8) for hf = 0, 1, each 4-byte group stored in the order {0, 2, 1, 3};
// [3072, 3328) the rows' 16 int8 scales (16 bytes per row), [3328, 3360) their FP16 d.
// Step s = 4hf + i covers elements 128hf + 32i + 8g + e (quant.rs:43-61).
struct FQ6K {
    static constexpr int KU = 256;
    struct Raw {
        uint4 a, b, c, sc;
        uint32_t d;
    };
    struct Prep {
        float d;
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *,
                                int K, int row, int u, int g) {
        const uint8_t *tb = wq + ((size_t)(row >> 4) * (size_t)(K / 256) + (size_t)u) * 3360u;
        const int rr = row & 15, lo = (16 * g + rr) * 16;
        r.a = ld16(tb + lo);
        r.b = ld16(tb + 1024 + lo);
        r.c = ld16(tb + 2048 + lo);
        r.sc = ld16(tb + 3072 + 16 * rr);
        r.d = *(const uint16_t *)(tb + 3328 + 2 * rr);
    }
    __device__ static void prep(const Raw &r, Prep &p, int) { p.d = h2f(r.d); }
    __device__ static int kidx(int s, int g) { return 32 * s + 8 * g; }
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int g, float v[8]) {
        const int hf = s >> 2, i = s & 3;
        const uint32_t w[12] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y,
                                r.b.z, r.b.w, r.c.x, r.c.y, r.c.z, r.c.w};
        const uint32_t sw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
        const int qi = 2 * (2 * hf + (i & 1));
        const int nib = 4 * (i >> 1);
        const int hi = 8 + 2 * hf;
        const int grp = 8 * hf + 2 * i + (g >> 1);
        const int32_t sc = (int32_t)(int8_t)((sw[grp >> 2] >> (8 * (grp & 3))) & 0xffu);
        const float scale = p.d * (float)sc;  // exact: 11 x 8 significant bits
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // the four 6-bit values q of one word, a byte each (q - 32 is quant.rs's value)
            uint32_t q6 = ((w[qi + h] >> nib) & 0x0f0f0f0fu) | (((w[hi + h] >> (2 * i)) & 0x03030303u) << 4);
            asm("" : "+v"(q6));  // one v_cvt_f32_ubyteN per byte
#pragma unroll
            for (int e = 4 * h; e < 4 * h + 4; ++e) {
                const int pos = ((e & 1) << 1) | ((e >> 1) & 1);  // stored byte of element e & 3
                // (d * sc) * (q - 32) as quant.rs evaluates it (the subtraction is exact; a
                // fused form would turn quant.rs's -0 for q = 32 and a negative scale into +0)
                v[e] = scale * ((float)((q6 >> (8 * pos)) & 0xffu) - 32.f);
            }
        }
    }
};

// Q6_K with the value s (q - 32) formed as fma(FP16 q - 32, s, -0): v_perm and one packed FP16
// subtraction make q - 32 for two elements, and one v_fma_mix_f32 per element replaces a
// conversion and a multiply. Bitwise the same values as FQ6K (signed zeros, infinities and NaN
// included). Used where it leaves the register count unchanged: the 8-wave 64 x 64 tile (down
// projection 85.6 against 88.8 us); on the 32 x 64 tile it costs 32 VGPRs and a wave per SIMD.
struct FQ6KMix : FQ6K {
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int g, float v[8]) {
        const int hf = s >> 2, i = s & 3;
        const uint32_t w[12] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y,
                                r.b.z, r.b.w, r.c.x, r.c.y, r.c.z, r.c.w};
        const uint32_t sw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
        const int qi = 2 * (2 * hf + (i & 1));
        const int nib = 4 * (i >> 1);
        const int hi = 8 + 2 * hf;
        const int grp = 8 * hf + 2 * i + (g >> 1);
        const int32_t sc = (int32_t)(int8_t)((sw[grp >> 2] >> (8 * (grp & 3))) & 0xffu);
        const float scale = p.d * (float)sc;
        const float nz = opaque_neg_zero();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t q6 = ((w[qi + h] >> nib) & 0x0f0f0f0fu) | (((w[hi + h] >> (2 * i)) & 0x03030303u) << 4);
            const h16x2 lo = bytes_f16_minus<0x05020500u>(q6, 0xe420e420u);  // q - 32
            const h16x2 up = bytes_f16_minus<0x05030501u>(q6, 0xe420e420u);
            v[4 * h + 0] = __builtin_fmaf((float)lo[0], scale, nz);
            v[4 * h + 1] = __builtin_fmaf((float)lo[1], scale, nz);
            v[4 * h + 2] = __builtin_fmaf((float)up[0], scale, nz);
            v[4 * h + 3] = __builtin_fmaf((float)up[1], scale, nz);
        }
    }
};

// Q8_0, device layout: 16-row tiles, per 64 k (two blocks) 1088 bytes: [0, 1024) lane 16g + r
// holds row r's block-0 elements 8g .. 8g+7 then its block-1 elements 8g .. 8g+7, as q + 128
// (the quant byte xor 0x80), in the order {0, 2, 1, 3} within each 4-byte group; [1024, 1088)
// the rows' two FP16 scales (4 bytes per row). Step s (0, 1) is block s; elements 32s + 8g + e
// (quant.rs:75-80).
struct FQ8_0 {
    static constexpr int KU = 64;
    struct Raw {
        uint4 q;
        uint32_t d2;
    };
    struct Prep {
        float d[2];
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *,
                                int K, int row, int u, int g) {
        const uint8_t *tb = wq + ((size_t)(row >> 4) * (size_t)(K / 64) + (size_t)u) * 1088u;
        const int rr = row & 15;
        r.q = ld16(tb + (16 * g + rr) * 16);
        r.d2 = *(const uint32_t *)(tb + 1024 + 4 * rr);
    }
    __device__ static void prep(const Raw &r, Prep &p, int) {
        p.d[0] = h2f(r.d2);
        p.d[1] = h2f(r.d2 >> 16);
    }
    __device__ static int kidx(int s, int g) { return 32 * s + 8 * g; }
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int, float v[8]) {
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        const float d = p.d[s];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int pos = ((e & 1) << 1) | ((e >> 1) & 1);  // stored byte of element e & 3
            // stored byte b = q + 128; b - 128 is exact, and d * q keeps quant.rs's signed zeros
            v[e] = d * ((float)((w[2 * s + (e >> 2)] >> (8 * pos)) & 0xffu) - 128.f);
        }
    }
};

// Q8_0 the same way (b - 128 = q as FP16, then fma(q, d, -0)); bitwise FQ8_0's values. Used by
// the 8-wave 64 x 64 and the 32 x 64 tiles (2-3 % faster at unchanged registers).
struct FQ8_0Mix : FQ8_0 {
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int, float v[8]) {
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        const float d = p.d[s];
        const float nz = opaque_neg_zero();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const h16x2 lo = bytes_f16_minus<0x05020500u>(w[2 * s + h], 0xe480e480u);  // b - 128
            const h16x2 up = bytes_f16_minus<0x05030501u>(w[2 * s + h], 0xe480e480u);
            v[4 * h + 0] = __builtin_fmaf((float)lo[0], d, nz);
            v[4 * h + 1] = __builtin_fmaf((float)lo[1], d, nz);
            v[4 * h + 2] = __builtin_fmaf((float)up[0], d, nz);
            v[4 * h + 3] = __builtin_fmaf((float)up[1], d, nz);
        }
    }
};

// Q5_0, device layout: per 64 k (two blocks) 32 quant bytes; bytes 16hb..16hb+15 hold
// block0 qs[8hb, +8) then block1 qs[8hb, +8); the h region holds each block's 32 high bits,
// the d region its FP16 scale. Lane group g holds elements 8g + e of each block: qs byte
// 8(g%2) + e, nibble g/2, high bit 8g + e (quant.rs:63-73).
struct FQ5_0 {
    static constexpr int KU = 64;
    struct Raw {
        uint4 q;
        uint2 h;
        uint32_t d2;
    };
    struct Prep {
        float d[2];
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *wh, const uint8_t *wd,
                                int K, int row, int u, int g) {
        const size_t ch = (size_t)row * (size_t)(K / 64) + (size_t)u;
        r.q = ld16(wq + ch * 32u + 16 * (g & 1));
        r.h = *(const uint2 *)(wh + ch * 8u);
        r.d2 = *(const uint32_t *)(wd + ch * 4u);
    }
    __device__ static void prep(const Raw &r, Prep &p, int) {
        p.d[0] = h2f(r.d2);
        p.d[1] = h2f(r.d2 >> 16);
    }
    __device__ static int kidx(int s, int g) { return 32 * s + 8 * g; }
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int g, float v[8]) {
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        const uint32_t qh = s ? r.h.y : r.h.x;
        const int nib = 4 * (g >> 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t lo = (w[2 * s + (e >> 2)] >> (8 * (e & 3) + nib)) & 15u;
            const uint32_t hb = (qh >> (8 * g + e)) & 1u;
            v[e] = p.d[s] * (float)((int32_t)(lo | (hb << 4)) - 16);
        }
    }
};

// Row-major FP16 weights [rows][K]: step s covers elements 32s + 8g + e of each 64-k unit.
struct FF16 {
    static constexpr int KU = 64;
    struct Raw {
        uint4 a, b;
    };
    struct Prep {};
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *,
                                int K, int row, int u, int g) {
        const uint8_t *base = wq + ((size_t)row * (size_t)K + 64u * (size_t)u) * 2u;
        r.a = ld16(base + 16 * g);
        r.b = ld16(base + 64 + 16 * g);
    }
    __device__ static void prep(const Raw &, Prep &, int) {}
    __device__ static int kidx(int s, int g) { return 32 * s + 8 * g; }
    __device__ static void frag_f32(const Raw &r, const Prep &, int s, int, float v[8]) {
        const uint4 q = s ? r.b : r.a;
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = h2f(w[e >> 1] >> (16 * (e & 1)));
    }
};

template <class F>
__device__ __forceinline__ f16x8 frag_f16(const typename F::Raw &r, const typename F::Prep &p,
                                          int s, int g) {
    float v[8];
    F::frag_f32(r, p, s, g, v);
    return pack8(v);
}

// ---------------------------------------------------------------------------------------------
// Activation staging: FP16 rows [m0, m0 + rows) x k [k0, k0 + kl) -> LDS, row stride `stride`
// (grouped: sorted positions m0 .. m0 + rows, each reading input row ids[s] / in_div). BF16 and
// FP32 rows reach the generic kernel as FP16 rows prescaled by jv_pack_x (rowmajor).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void stage_rows(const QmmParams &p, _Float16 *lds, int m0, int rows,
                                           int k0, int kl, int stride) {
    const int per_row = kl >> 3;
    const int total = rows * per_row;
    for (int i = threadIdx.x; i < total; i += kThreads) {
        const int r = i / per_row;
        const int c8 = i - r * per_row;
        const int xr = p.grouped ? (int)(p.ids[m0 + r] / (uint32_t)p.in_div) : m0 + r;
        const size_t src = (size_t)xr * (size_t)p.ldx + (size_t)(k0 + 8 * c8);
        *(uint4 *)(lds + r * stride + 8 * c8) = *(const uint4 *)((const uint16_t *)p.x + src);
    }
}

// ---------------------------------------------------------------------------------------------
// The product kernel. Grid: (N / (4*16*NT), ceil(M / (16*MT)), splits), 256 threads.
// ---------------------------------------------------------------------------------------------
template <class F, int MT, int NT>
__device__ __forceinline__ void qmm_body(const QmmParams &p) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int n_base = (int)blockIdx.x * (kWaves * 16 * NT) + wave * 16 * NT;
    int m0 = (int)blockIdx.y * 16 * MT;
    int rows_real = min(16 * MT, p.M - m0);
    int wrow0 = 0;  // first weight row (the expert's in grouped mode)
    if (p.grouped) {
        const int job = blockIdx.y;
        if (job >= (int)p.jobs[0]) return;  // the whole workgroup, before any barrier
        const int expert = (int)p.jobs[1 + 2 * job];
        m0 = (int)p.jobs[2 + 2 * job];
        rows_real = min(min((int)p.offsets[expert + 1] - m0, p.rows_cap), 16 * MT);
        wrow0 = expert * p.N;
    }
    const bool active = n_base < p.N;
    const int stride = p.kc + kLdsPad;

    const int U = p.K / F::KU;
    const int z = blockIdx.z;
    const int u_first = (int)((int64_t)z * U / p.splits);
    const int u_last = (int)((int64_t)(z + 1) * U / p.splits);
    const int kc_units = p.kc / F::KU;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    typename F::Raw cur[NT], nxt[NT];
    if (active && u_first < u_last) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            F::load(cur[t], p.wq, p.wh, p.wd, p.K, wrow0 + n_base + 16 * t + r16, u_first, g);
    }

    int chunk_u0 = u_first;
    for (int u = u_first; u < u_last; ++u) {
        if ((u - u_first) % kc_units == 0) {
            chunk_u0 = u;
            const int kl = min(kc_units, u_last - u) * F::KU;
            lds_barrier();
            stage_rows(p, lds, m0, rows_real, u * F::KU, kl, stride);
            lds_barrier();
        }
        if (active) {
            if (u + 1 < u_last) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    F::load(nxt[t], p.wq, p.wh, p.wd, p.K, wrow0 + n_base + 16 * t + r16, u + 1, g);
            }
            typename F::Prep pp[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) F::prep(cur[t], pp[t], g);
            const int ubase = (u - chunk_u0) * F::KU;
#pragma unroll
            for (int s = 0; s < F::KU / 32; ++s) {
                f16x8 b[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) b[t] = frag_f16<F>(cur[t], pp[t], s, g);
                const int kk = ubase + F::kidx(s, g);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int lr = mt * 16 + r16;
                    f16x8 a = {};
                    if (lr < rows_real) a = *(const f16x8 *)(lds + lr * stride + kk);
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[t], acc[mt][t], 0, 0, 0);
                }
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) cur[t] = nxt[t];
        }
    }

    if (!active) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lr = mt * 16 + 4 * g + i;
            if (lr >= rows_real) continue;
            const int row = p.grouped ? (int)p.ids[m0 + lr] : m0 + lr;
            // the input row's range factor (prescaled FP16 rows; exact, a power of two)
            const float rs = p.rscale ? p.rscale[p.grouped ? row / p.in_div : row] : 1.f;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int col = n_base + 16 * t + r16;
                const float v = acc[mt][t][i] * rs;
                if (p.splits > 1) {
                    float *o = (float *)p.out + (int64_t)z * p.split_stride;
                    o[(size_t)row * (size_t)p.ldo + (size_t)col] = v;
                } else if (p.out_type == 0) {
                    ((float *)p.out)[(size_t)row * (size_t)p.ldo + (size_t)col] = v;
                } else {
                    ((uint16_t *)p.out)[(size_t)row * (size_t)p.ldo + (size_t)col] = (uint16_t)f2bf(v);
                }
            }
        }
    }
}

// Decode probe: each wave decodes 16 weight rows; lane (r, g) writes its 8 values per step.
template <class F>
__device__ __forceinline__ void dequant_body(const DequantParams &p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int lr = ((int)blockIdx.x * kWaves + wave) * 16 + r16;
    if (lr >= p.rows) return;
    const int row = p.row0 + lr;
    const int U = p.K / F::KU;
    for (int u = 0; u < U; ++u) {
        typename F::Raw raw;
        typename F::Prep pp;
        F::load(raw, p.wq, p.wh, p.wd, p.K, row, u, g);
        F::prep(raw, pp, g);
#pragma unroll
        for (int s = 0; s < F::KU / 32; ++s) {
            float v[8];
            F::frag_f32(raw, pp, s, g, v);
            const size_t o = (size_t)lr * (size_t)p.K + (size_t)(u * F::KU + F::kidx(s, g));
            if (p.f16_out) {
                *(f16x8 *)((_Float16 *)p.out + o) = pack8(v);
            } else {
                float *dst = (float *)p.out + o;
                *(float4 *)dst = float4{v[0], v[1], v[2], v[3]};
                *(float4 *)(dst + 4) = float4{v[4], v[5], v[6], v[7]};
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Small-row Q4_K product (M <= 16) with exact integer weights.
//
// Per block and weight row, out += d * sum_j s'_j S_j - sum_j (1024 d s'_j + dmin m_j) X_j, where
//   S_j = sum_e x_e * (1024 + q_e) over sub-block j (32 elements, one MFMA 16x16x32 f16), the
//         FP16 operand 1024 + q being exact and built with one and-or on the bit pattern
//         0x6400 (= 1024.0): low nibbles give 1024 + q, high nibbles 1024 + 16 q;
//   s'_j = s_j for even j and s_j / 16 for odd j (high nibbles carry 16 q);
//   X_j = sum of the activations over sub-block j, prepared with the LDS staging;
//   the bias terms are one FP32 MFMA 16x16x4 pair (k = sub-block).
// This equals sum_e x_e * (d*s_j*q_e - dmin*m_j), the quant.rs:25-41 weights times x, up to FP32
// rounding of the sums: the products x * (1024 + q) are exact, and the 1024 X_j term cancels
// against the sums' 1024 x_e parts to FP32 rounding. The device layout stores each 4-byte group of
// quant bytes in the order {0, 2, 1, 3}, so (w & 0x000f000f) holds two consecutive elements and
// the activation fragments are read in natural order.
// ---------------------------------------------------------------------------------------------
// Q4_K (scale, min) of sub-blocks 2g and 2g+1, branch-free (quant.rs:14-23): lane groups
// 0-1 hold sub-blocks 0-3 (low form), groups 2-3 sub-blocks 4-7 (high form).
__device__ __forceinline__ void q4k_pair_scales(const uint4 &hd, int g, uint32_t sc[2], uint32_t mn[2]) {
    const bool hi = g >= 2;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int sh = 16 * (g & 1) + 8 * h;  // 8 * ((2g + h) & 3)
        const uint32_t a = hd.y >> sh, b = hd.z >> sh, c = hd.w >> sh;
        const uint32_t sc_lo = a & 63u, mn_lo = b & 63u;
        const uint32_t sc_hi = (c & 15u) | ((a >> 2) & 48u);
        const uint32_t mn_hi = ((c >> 4) & 15u) | ((b >> 2) & 48u);
        sc[h] = hi ? sc_hi : sc_lo;
        mn[h] = hi ? mn_hi : mn_lo;
    }
}

// One Q4_K block of a 16-row tile as one lane holds it: quant bytes as FQ4K::load reads them,
// and one dword of the heads instead of a whole head. Lane 16g + r loads dword g of row r's
// 16-byte head, so the wave reads the 256 head bytes once (a 16-byte load replicated over the
// four lane groups costs about as much load bandwidth as 1 KB of quants).
struct Q4KItem {
    uint4 q0, q1;
    uint32_t hv;
};

__device__ __forceinline__ void q4k_item_load(Q4KItem &it, const uint8_t *wq, int K, int tile,
                                              int u, int g, int r) {
    const uint8_t *tb = wq + ((size_t)tile * (size_t)(K / 256) + (size_t)u) * 2304u;
    const uint32_t lq = (uint32_t)(16 * g + r) * 16u, lh = 2048u + (uint32_t)(r * 16 + 4 * g);
    it.q0 = ld16(tb + lq);
    it.q1 = ld16(tb + 1024u + lq);
    it.hv = *(const uint32_t *)(tb + lh);
}

// All four head dwords of row r in every lane group, from lane 16g + r holding dword g.
// permlane16_swap exchanges odd 16-lane rows of its first operand with even rows of its
// second; permlane32_swap exchanges the upper 32 lanes of the first with the lower 32 of the
// second (gfx950).
__device__ __forceinline__ uint4 q4k_head_gather(uint32_t hv) {
    const auto x = __builtin_amdgcn_permlane16_swap(hv, hv, false, false);  // {d0,d0,d2,d2}, {d1,d1,d3,d3}
    const auto e = __builtin_amdgcn_permlane32_swap(x[0], x[0], false, false);  // d0, d2 everywhere
    const auto o = __builtin_amdgcn_permlane32_swap(x[1], x[1], false, false);  // d1, d3 everywhere
    return uint4{(uint32_t)e[0], (uint32_t)o[0], (uint32_t)e[1], (uint32_t)o[1]};
}

// Stages columns [c0, c0 + ncols) of activation rows [0, M) for one wave: FP16 into
// xs[r * stride + c] and FP32 sums of each XG-column group (16 or 32) into Xs[r * xstride + c / XG].
// The wave's first XB 16-byte loads per lane are issued before `after()` (the weight loads),
// so waiting for them does not wait for the weights; later batches, if any, come after.
// Returns true in a lane that wrote a non-finite sum: some staged value of that sub-block was
// non-finite, which for finite BF16 and FP32 inputs means it overflowed the FP16 range.
template <int ACT, int XB, int XG, bool GRP = false, class After>
__device__ __forceinline__ bool stage_wave_cols(const QmmParams &p, int c0, int ncols, _Float16 *xs,
                                                int stride, float *Xs, int xstride, int lane,
                                                After after) {
    constexpr int EPL = ACT == 2 ? 4 : 8;  // elements per 16-byte load
    constexpr int LPC = 8 / EPL;           // loads per 8-element chunk
    constexpr int XC = XB / LPC;           // chunks held per lane at once
    const int per_row = ncols >> 3;
    const int total = p.M * per_row;  // 8-element chunks; a multiple of 4 (ncols % 32 == 0)
    // chunk i = row r, 8-column group c8: r = floor((i + 0.5) / per_row) through a float
    // reciprocal, exact for i < 2^22 (the rounding error stays below the 0.5 / per_row margin)
    const float rcp = 1.0f / (float)per_row;
    bool issued = false, nonfinite = false;
    for (int i0 = 0; i0 < total; i0 += XC * 64) {
        uint4 raw[XC][LPC];
        int rq[XC], cq[XC];
        const int nq = min(XC, (total - i0 + 63) >> 6);  // uniform: batches holding real chunks
#pragma unroll
        for (int q = 0; q < XC; ++q) {
            if (q >= nq) break;
            const int i = min(i0 + q * 64 + lane, total - 1);
            const int r = (int)(((float)i + 0.5f) * rcp);
            const int c8 = i - r * per_row;
            rq[q] = r;
            cq[q] = c8;
            // expert-grouped: row r of the job is input row ids[r] / in_div (ids = the job's first
            // sorted position)
            const int xr = GRP ? (int)(p.ids[r] / (uint32_t)p.in_div) : r;
            const size_t src = (size_t)xr * (size_t)p.ldx + (size_t)(c0 + 8 * c8);
#pragma unroll
            for (int hh = 0; hh < LPC; ++hh) {
                if (ACT == 2)
                    raw[q][hh] = *(const uint4 *)((const float *)p.x + src + 4 * hh);
                else
                    raw[q][hh] = *(const uint4 *)((const uint16_t *)p.x + src);
            }
        }
        if (!issued) {
            after();
            issued = true;
        }
#pragma unroll
        for (int q = 0; q < XC; ++q) {
            if (q >= nq) break;
            const int i = i0 + q * 64 + lane;
            float part = 0.f;
            int r = 0, c8 = 0;
            if (i < total) {
                r = rq[q];  // i is not clamped here
                c8 = cq[q];
                float v[8];
                if (ACT == 2) {
#pragma unroll
                    for (int hh = 0; hh < LPC; ++hh) {
                        v[4 * hh + 0] = __builtin_bit_cast(float, raw[q][hh].x);
                        v[4 * hh + 1] = __builtin_bit_cast(float, raw[q][hh].y);
                        v[4 * hh + 2] = __builtin_bit_cast(float, raw[q][hh].z);
                        v[4 * hh + 3] = __builtin_bit_cast(float, raw[q][hh].w);
                    }
                } else {
                    const uint32_t w[4] = {raw[q][0].x, raw[q][0].y, raw[q][0].z, raw[q][0].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] = ACT == 0 ? h2f(w[e]) : bf2f(w[e]);
                        v[2 * e + 1] = ACT == 0 ? h2f(w[e] >> 16) : bf2f(w[e] >> 16);
                    }
                }
                f16x8 h;
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = (_Float16)v[e];
                // FP32 sum of the FP16 values, two per dot-product step
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    part = __builtin_amdgcn_fdot2(f16x2{h[2 * e], h[2 * e + 1]}, f16x2{1.0f16, 1.0f16}, part, false);
                *(f16x8 *)(xs + r * stride + 8 * c8) = h;
            }
            // lanes 4q..4q+3 hold the four 8-element chunks of one 32-element sub-block
            part += __shfl_xor(part, 1);
            if (XG == 32) part += __shfl_xor(part, 2);
            if (i < total && (c8 & (XG / 8 - 1)) == 0) Xs[r * xstride + c8 / (XG / 8)] = part;
            nonfinite |= !__builtin_isfinite(part);
        }
    }
    if (!issued) after();
    return nonfinite;
}

// stage_wave_cols with the work shared by the W waves of a workgroup: the 8-element chunks are
// numbered row-major and wave w takes the 64-chunk batches w, w + W, w + 2W, ... Each chunk's
// values and sums are computed as in stage_wave_cols.
template <int ACT, int XB, int XG, int W, class After>
__device__ __forceinline__ bool stage_group_cols(const QmmParams &p, int c0, int ncols, _Float16 *xs,
                                                 int stride, float *Xs, int xstride, int lane,
                                                 int wave, After after) {
    constexpr int EPL = ACT == 2 ? 4 : 8;  // elements per 16-byte load
    constexpr int LPC = 8 / EPL;           // loads per 8-element chunk
    constexpr int XC = XB / LPC;           // chunks held per lane at once
    const int per_row = ncols >> 3;
    const int total = p.M * per_row;  // 8-element chunks; a multiple of 4 (ncols % 32 == 0)
    // chunk i = row r, 8-column group c8: r = floor((i + 0.5) / per_row) through a float
    // reciprocal, exact for i < 2^22 (the rounding error stays below the 0.5 / per_row margin)
    const float rcp = 1.0f / (float)per_row;
    bool issued = false, nonfinite = false;
    for (int i0 = 64 * wave; i0 < total; i0 += XC * 64 * W) {
        uint4 raw[XC][LPC];
        int rq[XC], cq[XC];
        const int nq = min(XC, (total - i0 + 64 * W - 1) / (64 * W));  // uniform: batches holding real chunks
#pragma unroll
        for (int q = 0; q < XC; ++q) {
            if (q >= nq) break;
            const int i = min(i0 + q * 64 * W + lane, total - 1);
            const int r = (int)(((float)i + 0.5f) * rcp);
            const int c8 = i - r * per_row;
            rq[q] = r;
            cq[q] = c8;
            const size_t src = (size_t)r * (size_t)p.ldx + (size_t)(c0 + 8 * c8);
#pragma unroll
            for (int hh = 0; hh < LPC; ++hh) {
                if (ACT == 2)
                    raw[q][hh] = *(const uint4 *)((const float *)p.x + src + 4 * hh);
                else
                    raw[q][hh] = *(const uint4 *)((const uint16_t *)p.x + src);
            }
        }
        if (!issued) {
            after();
            issued = true;
        }
#pragma unroll
        for (int q = 0; q < XC; ++q) {
            if (q >= nq) break;
            const int i = i0 + q * 64 * W + lane;
            float part = 0.f;
            int r = 0, c8 = 0;
            if (i < total) {
                r = rq[q];  // i is not clamped here
                c8 = cq[q];
                float v[8];
                if (ACT == 2) {
#pragma unroll
                    for (int hh = 0; hh < LPC; ++hh) {
                        v[4 * hh + 0] = __builtin_bit_cast(float, raw[q][hh].x);
                        v[4 * hh + 1] = __builtin_bit_cast(float, raw[q][hh].y);
                        v[4 * hh + 2] = __builtin_bit_cast(float, raw[q][hh].z);
                        v[4 * hh + 3] = __builtin_bit_cast(float, raw[q][hh].w);
                    }
                } else {
                    const uint32_t w[4] = {raw[q][0].x, raw[q][0].y, raw[q][0].z, raw[q][0].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] = ACT == 0 ? h2f(w[e]) : bf2f(w[e]);
                        v[2 * e + 1] = ACT == 0 ? h2f(w[e] >> 16) : bf2f(w[e] >> 16);
                    }
                }
                f16x8 h;
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = (_Float16)v[e];
                // FP32 sum of the FP16 values, two per dot-product step
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    part = __builtin_amdgcn_fdot2(f16x2{h[2 * e], h[2 * e + 1]}, f16x2{1.0f16, 1.0f16}, part, false);
                *(f16x8 *)(xs + r * stride + 8 * c8) = h;
            }
            // lanes 4q..4q+3 hold the four 8-element chunks of one 32-element sub-block
            part += __shfl_xor(part, 1);
            if (XG == 32) part += __shfl_xor(part, 2);
            if (i < total && (c8 & (XG / 8 - 1)) == 0) Xs[r * xstride + c8 / (XG / 8)] = part;
            nonfinite |= !__builtin_isfinite(part);
        }
    }
    if (!issued) after();
    return nonfinite;
}

// Power-of-two range scale of a row whose largest magnitude is `mx` (the reference's
// F16_ROW_LIMIT rule, crates/jevons-burn/src/kernels.rs:105, :120-130, with a power of two, so
// that the scaling is exact): 2^-e with e = floor(log2 mx) - 13 when mx > 16384, so that the
// scaled magnitudes stay below 2^14; 1 for smaller or non-finite maxima (a non-finite value
// stays non-finite in the product, as in the reference). Returns 2^-e and sets *inv = 2^e.
__device__ __forceinline__ float range_scale(float mx, float *inv) {
    if (!(mx > 16384.f) || !__builtin_isfinite(mx)) {
        *inv = 1.f;
        return 1.f;
    }
    const int e = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xffu) - 127 - 13;  // 1..114
    *inv = __builtin_bit_cast(float, (uint32_t)(127 + e) << 23);
    return __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
}

// The 8 activations of chunk (row xr, columns col .. col + 7) as FP32.
template <int ACT>
__device__ __forceinline__ void load_act8(const QmmParams &p, int xr, int col, float v[8]) {
    const size_t src = (size_t)xr * (size_t)p.ldx + (size_t)col;
    if (ACT == 2) {
        const float4 a = *(const float4 *)((const float *)p.x + src);
        const float4 b = *(const float4 *)((const float *)p.x + src + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 b = *(const uint4 *)((const uint16_t *)p.x + src);
        const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = ACT == 0 ? h2f(w[e]) : bf2f(w[e]);
            v[2 * e + 1] = ACT == 0 ? h2f(w[e] >> 16) : bf2f(w[e] >> 16);
        }
    }
}

// Stages row r of columns [c0, c0 + ncols) again, as stage_wave_cols does, but multiplied by the
// row's range_scale over those columns; one wave. Sc[r] receives the factor that undoes it. Runs
// only when a staged value overflowed the FP16 range (rows without values above 16384 get scale
// 1 and so the same values as the first staging).
template <int ACT, int XG, bool GRP>
__device__ __forceinline__ void stage_row_scaled(const QmmParams &p, int r, int c0, int ncols,
                                                 _Float16 *xs, int stride, float *Xs, int xstride,
                                                 float *Sc, int lane) {
    const int per_row = ncols >> 3;  // a multiple of 4
    const int xr = GRP ? (int)(p.ids[r] / (uint32_t)p.in_div) : r;
    float mx = 0.f;
    bool nf = false;
    for (int c = lane; c < per_row; c += 64) {
        float v[8];
        load_act8<ACT>(p, xr, c0 + 8 * c, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            nf |= !__builtin_isfinite(v[e]);
            mx = __builtin_fmaxf(mx, __builtin_fabsf(v[e]));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, off));
    float inv;
    const float scale = range_scale(__any(nf) ? __builtin_inff() : mx, &inv);
    if (lane == 0) Sc[r] = inv;
    for (int c00 = 0; c00 < per_row; c00 += 64) {  // uniform trip count: the sums shuffle
        const int c = c00 + lane;
        float part = 0.f;
        if (c < per_row) {
            float v[8];
            load_act8<ACT>(p, xr, c0 + 8 * c, v);
            f16x8 h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (_Float16)(v[e] * scale);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                part = __builtin_amdgcn_fdot2(f16x2{h[2 * e], h[2 * e + 1]}, f16x2{1.0f16, 1.0f16}, part, false);
            *(f16x8 *)(xs + r * stride + 8 * c) = h;
        }
        part += __shfl_xor(part, 1);
        if (XG == 32) part += __shfl_xor(part, 2);
        if (c < per_row && (c & (XG / 8 - 1)) == 0) Xs[r * xstride + c / (XG / 8)] = part;
    }
}

// A wave's staging of its columns for all p.M rows (stage_wave_cols), redone row by row with range
// scales when some value overflowed FP16. Returns whether it was (wave-uniform); then Sc[r] holds
// the factor that undoes row r's scale.
template <int ACT, int XB, int XG, bool GRP, class After>
__device__ __forceinline__ bool stage_wave_checked(const QmmParams &p, int c0, int ncols, _Float16 *xs,
                                                   int stride, float *Xs, int xstride, float *Sc,
                                                   int lane, After after) {
    const bool nf = stage_wave_cols<ACT, XB, XG, GRP>(p, c0, ncols, xs, stride, Xs, xstride, lane, after);
    if (!__any(nf)) return false;
    for (int r = 0; r < p.M; ++r)
        stage_row_scaled<ACT, XG, GRP>(p, r, c0, ncols, xs, stride, Xs, xstride, Sc, lane);
    return true;
}

// Rows of the small-row products are spread over the four lane groups: with RPG = ceil(M / 4)
// rows per group, row m is MFMA row 4 (m / RPG) + m % RPG, so lane group g holds rows
// g RPG .. g RPG + RPG - 1 in accumulator elements 0 .. RPG - 1, and the per-row arithmetic
// after each MFMA covers RPG elements instead of 4 (M = 2 to 4 cost what M = 1 costs). Each
// output element is the same MFMA and FMA chain wherever its row sits, so the bits do not depend
// on M. The activation row that MFMA row r reads (rows with r % 4 >= RPG feed accumulator
// elements that are never stored, and read a real row):
__device__ __forceinline__ int spread_row(int r, int rpg, int M) {
    return min((r >> 2) * rpg + min(r & 3, rpg - 1), M - 1);
}
// Output row of accumulator element i of lane group g, or -1 for an element holding no row.
__device__ __forceinline__ int spread_out(int g, int i, int rpg, int M) {
    const int m = g * rpg + i;
    return i < rpg && m < M ? m : -1;
}

// ---------------------------------------------------------------------------------------------
// Greedy epilogue of the vocabulary projection (lm_head, soft cap and greedy fused:
// crates/jevons-gemma4-diffusion/src/model.rs:1194-1204 and gpu/ops.rs:750-758, then
// crates/jevons-core/src/model.rs:207-219 on each row): outputs are soft-capped before they are
// stored, and each workgroup leaves per row the largest value of its columns and that value's
// first column, for jv_argmax_final.
// ---------------------------------------------------------------------------------------------
// (v, i) replaces (bv, bi) if larger, or equal with a lower index: greedy's first maximum.
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// tanh for the soft cap, odd: below |y| = 0.625 the series form y + y^3 Q(y^2), with Q of
// degree 5 fitted by least squares to (tanh y / y - 1) / y^2 on [0, 0.625^2] (fit error 5e-9
// relative; softcap_tanh_fit.py beside this file recomputes it); above, tanh |y| = 1 - 2 / (e^(2|y|) + 1) through the hardware 2^x and
// reciprocal (e^(2|y|) = 2^(2 log2(e) |y|)). Within 2 ulp of tanh in float32 simulation and
// a few ulp on the device (the tests hold it to 6), at a third of the library call's
// instructions. +-inf give +-1, NaN stays NaN.
__device__ __forceinline__ float cap_tanh(float y) {
    const float a = __builtin_fabsf(y), t = y * y;
    float q = 1.618547598e-03f;
    q = __builtin_fmaf(q, t, -7.621073630e-03f);
    q = __builtin_fmaf(q, t, 2.148471028e-02f);
    q = __builtin_fmaf(q, t, -5.390961096e-02f);
    q = __builtin_fmaf(q, t, 1.333293766e-01f);
    q = __builtin_fmaf(q, t, -3.333332539e-01f);
    const float small = __builtin_fmaf(y * t, q, y);
    const float e = __builtin_amdgcn_exp2f(a * 2.885390082f);
    const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    return a < 0.625f ? small : __builtin_copysignf(big, y);
}

// The soft cap of one output value, cap tanh(v / cap), the same expression in jv_softcap and in
// the greedy epilogue; cap 0 leaves it.
__device__ __forceinline__ float soft_capped(float v, float cap) {
    return cap > 0.f ? cap * cap_tanh(v * (1.0f / cap)) : v;
}

// A (value, column) pair as one 64-bit key whose unsigned maximum is greedy's pick: the value's
// bits mapped to an unsigned order (negative values inverted, positive ones with the sign bit
// set), above the inverted column, so that equal values keep the lowest column. -0 is taken as
// +0, which compares equal to it.
__device__ __forceinline__ uint64_t greedy_key(float v, int col) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v == 0.f ? 0.f : v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(~(uint32_t)col);
}

// Largest value, its first column and whether any value was not finite, over the columns of one
// output row that a lane (then a lane group, a wave, a workgroup) stores.
struct Greedy {
    float v;
    int i;
    int bad;
    __device__ static Greedy none() { return Greedy{-__builtin_inff(), 0x7fffffff, 0}; }
    __device__ void add(float x, int col) {
        bad |= !__builtin_isfinite(x);
        better(v, i, x, col);
    }
    __device__ void merge(const Greedy &o) {
        better(v, i, o.v, o.i);
        bad |= o.bad;
    }
    // over the 16 lanes of the lane group (the lanes that hold the same output rows)
    __device__ void group16() {
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const float ov = __shfl_xor(v, off);
            const int oi = __shfl_xor(i, off);
            const int ob = __shfl_xor(bad, off);
            better(v, i, ov, oi);
            bad |= ob;
        }
    }
    // this row's result folded into its key or flag (agent-scope atomics, no return)
    __device__ void fold(uint64_t *key, uint32_t *bad_row) const {
        if (bad)
            __hip_atomic_fetch_or(bad_row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            __hip_atomic_fetch_max(key, greedy_key(v, i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
};

// After a product whose workgroups folded their rows into the greedy keys (Greedy::fold): each
// row's column (-1 for a flagged row), and the keys and flags zeroed for the next launch. Grid:
// ceil(M / 256) x 256 threads.
extern "C" __global__ __launch_bounds__(256) void jv_greedy_finish(uint64_t *key, uint32_t *bad, int32_t *out,
                                                                  int M) {
    const int r = (int)(blockIdx.x * 256 + threadIdx.x);
    if (r >= M) return;
    const uint64_t k = key[r];
    out[r] = bad[r] ? -1 : (int32_t)~(uint32_t)k;
    key[r] = 0;
    bad[r] = 0;
}

// Formats whose scale groups are 16 columns (Q6_K) run each 32-k step as MFMA rows of activation
// rows masked to one half of the step: MFMA row 4q + 2a + h reads activation row q rpg + a (the
// row of accumulator element a of lane group q) in lane groups 2h, 2h + 1 and the zero row in
// the others, so the element of row 4q + 2a + h is the half-h sum of that row. Up to 8 rows (two
// per lane group) fit one MFMA. The lane's A pointer for that layout:
__device__ __forceinline__ const _Float16 *half_row(const _Float16 *xs, const _Float16 *zrow, int stride,
                                                  int r, int g, int M) {
    const int rpg = (M + 3) >> 2;
    const int row = min((r >> 2) * rpg + min((r >> 1) & 1, rpg - 1), M - 1);
    return ((g >> 1) == (r & 1)) ? xs + row * stride : zrow;
}

// Multiplies a lane's accumulator (lane group g's rows) by the rows' range factors.
__device__ __forceinline__ void unscale_rows(f32x4 &a, const float *Sc, int g, int M) {
    const int rpg = (M + 3) >> 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] *= Sc[min(g * rpg + min(i, rpg - 1), M - 1)];
}

// One block against activations staged in LDS, with the scale arithmetic regrouped to cut
// vector ALU work (the kernel is bound by it once the loads are in flight):
//   out += d * (sum_even s_j S_j + (sum_odd s_j S_j) / 16) - sum_j (1024 d s'_j + dmin m_j) X_j,
// the eight 6-bit scales unpacked with byte masks, and the bias terms of sub-blocks g and
// 4 + g (lane group g; k index g of the two FP32 MFMAs 16x16x4) extracted with lane-variable
// shifts sh = 8 g. kfac = -1024 for even g, -64 for odd g (sub-blocks g and 4 + g hold high
// nibbles, 16 q, when g is odd). The result equals quant.rs:25-41's weights times x up to FP32
// rounding of the sums; each output row's arithmetic is the same for every M.
template <int MV>
__device__ __forceinline__ void q4k_block_fast(const Q4KItem &cur, const _Float16 *xrow,
                                               const float *Xrow, int ul, int g, uint32_t sh,
                                               float kfac, f32x4 &acc) {
    const uint4 hd = q4k_head_gather(cur.hv);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    // scale bytes: y = q[0..3], z = q[4..7], w = q[8..11] (quant.rs:14-23)
    uint32_t s_lo = hd.y & 0x3f3f3f3fu;                                         // s_0..s_3
    asm("" : "+v"(s_lo));  // opaque: each byte converts with one v_cvt_f32_ubyteN
    const uint32_t s_hi = ((hd.y >> 2) & 0x30303030u) | (hd.w & 0x0f0f0f0fu);    // s_4..s_7
    const uint32_t m_hi = ((hd.z >> 2) & 0x30303030u) | ((hd.w >> 4) & 0x0f0f0f0fu);  // m_4..m_7
    const float sg = (float)((s_lo >> sh) & 0xffu), s4g = (float)((s_hi >> sh) & 0xffu);
    const float mg = (float)((hd.z >> sh) & 63u), m4g = (float)((m_hi >> sh) & 0xffu);
    const float kd = kfac * d;
    const float cA = __builtin_fmaf(kd, sg, -(dmin * mg));
    const float cB = __builtin_fmaf(kd, s4g, -(dmin * m4g));
    float sj[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        sj[k] = (float)((s_lo >> (8 * k)) & 0xffu);
        sj[4 + k] = (float)((s_hi >> (8 * k)) & 0xffu);
    }
    uint32_t magic = 0x64006400u;
    asm("" : "+v"(magic));
    const int kb = ul * 256 + 8 * g;
    const uint32_t w[8] = {cur.q0.x, cur.q0.y, cur.q0.z, cur.q0.w, cur.q1.x, cur.q1.y, cur.q1.z, cur.q1.w};
    float ve[MV], vo[MV];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        f32x4 S[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = 4 * hf + q;
            const uint32_t wa = w[j & ~1], wb = w[(j & ~1) + 1];
            const uint32_t mask = (j & 1) ? 0x00f000f0u : 0x000f000fu;
            uint4 bq;
            bq.x = (wa & mask) | magic;
            bq.y = ((wa >> 8) & mask) | magic;
            bq.z = (wb & mask) | magic;
            bq.w = ((wb >> 8) & mask) | magic;
            S[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8 *)(xrow + kb + 32 * j),
                                                          __builtin_bit_cast(f16x8, bq),
                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MV; ++i) {
            if (hf == 0) {
                ve[i] = sj[0] * S[0][i];
                vo[i] = sj[1] * S[1][i];
            } else {
                ve[i] = __builtin_fmaf(sj[4], S[0][i], ve[i]);
                vo[i] = __builtin_fmaf(sj[5], S[1][i], vo[i]);
            }
            ve[i] = __builtin_fmaf(sj[4 * hf + 2], S[2][i], ve[i]);
            vo[i] = __builtin_fmaf(sj[4 * hf + 3], S[3][i], vo[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < MV; ++i) acc[i] = __builtin_fmaf(d, __builtin_fmaf(vo[i], 0.0625f, ve[i]), acc[i]);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Xrow[ul * 8 + g], cA, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Xrow[ul * 8 + 4 + g], cB, acc, 0, 0, 0);
}

// q4k_block_fast with the unit's activation fragments A[j] and sums xa = X_g, xb = X_{4+g} in
// registers: the same instructions on the same values, so the same bits.
template <int MV>
__device__ __forceinline__ void q4k_block_regs(const Q4KItem &cur, const f16x8 A[8], float xa, float xb,
                                               uint32_t sh, float kfac, f32x4 &acc) {
    const uint4 hd = q4k_head_gather(cur.hv);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    // scale bytes: y = q[0..3], z = q[4..7], w = q[8..11] (quant.rs:14-23)
    uint32_t s_lo = hd.y & 0x3f3f3f3fu;                                         // s_0..s_3
    asm("" : "+v"(s_lo));  // opaque: each byte converts with one v_cvt_f32_ubyteN
    const uint32_t s_hi = ((hd.y >> 2) & 0x30303030u) | (hd.w & 0x0f0f0f0fu);    // s_4..s_7
    const uint32_t m_hi = ((hd.z >> 2) & 0x30303030u) | ((hd.w >> 4) & 0x0f0f0f0fu);  // m_4..m_7
    const float sg = (float)((s_lo >> sh) & 0xffu), s4g = (float)((s_hi >> sh) & 0xffu);
    const float mg = (float)((hd.z >> sh) & 63u), m4g = (float)((m_hi >> sh) & 0xffu);
    const float kd = kfac * d;
    const float cA = __builtin_fmaf(kd, sg, -(dmin * mg));
    const float cB = __builtin_fmaf(kd, s4g, -(dmin * m4g));
    float sj[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        sj[k] = (float)((s_lo >> (8 * k)) & 0xffu);
        sj[4 + k] = (float)((s_hi >> (8 * k)) & 0xffu);
    }
    uint32_t magic = 0x64006400u;
    asm("" : "+v"(magic));
    const uint32_t w[8] = {cur.q0.x, cur.q0.y, cur.q0.z, cur.q0.w, cur.q1.x, cur.q1.y, cur.q1.z, cur.q1.w};
    float ve[MV], vo[MV];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        f32x4 S[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = 4 * hf + q;
            const uint32_t wa = w[j & ~1], wb = w[(j & ~1) + 1];
            const uint32_t mask = (j & 1) ? 0x00f000f0u : 0x000f000fu;
            uint4 bq;
            bq.x = (wa & mask) | magic;
            bq.y = ((wa >> 8) & mask) | magic;
            bq.z = (wb & mask) | magic;
            bq.w = ((wb >> 8) & mask) | magic;
            S[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[j], __builtin_bit_cast(f16x8, bq),
                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MV; ++i) {
            if (hf == 0) {
                ve[i] = sj[0] * S[0][i];
                vo[i] = sj[1] * S[1][i];
            } else {
                ve[i] = __builtin_fmaf(sj[4], S[0][i], ve[i]);
                vo[i] = __builtin_fmaf(sj[5], S[1][i], vo[i]);
            }
            ve[i] = __builtin_fmaf(sj[4 * hf + 2], S[2][i], ve[i]);
            vo[i] = __builtin_fmaf(sj[4 * hf + 3], S[3][i], vo[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < MV; ++i) acc[i] = __builtin_fmaf(d, __builtin_fmaf(vo[i], 0.0625f, ve[i]), acc[i]);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, cA, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xb, cB, acc, 0, 0, 0);
}

// Q4_K as a small-row format: item = one 256-element block of a 16-row tile.
struct GQ4K {
    static constexpr int KU = 256;  // K per item
    static constexpr int XG = 32;   // activation sum group
    static constexpr bool kZeroRow = false;
    typedef Q4KItem Item;
    struct Lane {
        uint32_t sh;
        float kfac;
    };
    __device__ static Lane lane_consts(int g) {
        return Lane{8u * (uint32_t)g, (g & 1) ? -64.f : -1024.f};
    }
    __device__ static void load(Item &it, const QmmParams &p, int tile, int u, int g, int r) {
        q4k_item_load(it, p.wq, p.K, tile, u, g, r);
    }
    template <int MV>
    __device__ static void block(const Item &it, const _Float16 *xrow, const _Float16 *, const float *Xrow,
                                 int ul, int g, const Lane &c, f32x4 &acc) {
        q4k_block_fast<MV>(it, xrow, Xrow, ul, g, c.sh, c.kfac, acc);
    }
};

// Q8_0 as a small-row format: item = 64 k (two blocks) of a 16-row tile. Block b is one MFMA on
// the FP16 operands q: 0x6400 | (q + 128) (the stored byte) is 1152 + q, and one packed FP16
// subtraction of 1152 leaves q exactly; the sum is scaled by d_b. The products x q are exact,
// so this equals quant.rs:75-80's weights times x up to FP32 rounding, with no bias term.
struct GQ8_0 {
    static constexpr _Float16 kOff = (_Float16)-1152.0f;
    static constexpr int KU = 64;
    static constexpr int XG = 32;
    static constexpr bool kZeroRow = false;
    struct Item {
        uint4 q;
        uint32_t d2;
    };
    struct Lane {};
    __device__ static Lane lane_consts(int) { return Lane{}; }
    __device__ static void load(Item &it, const QmmParams &p, int tile, int u, int g, int r) {
        const uint8_t *tb = p.wq + ((size_t)tile * (size_t)(p.K / 64) + (size_t)u) * 1088u;
        it.q = ld16(tb + (16 * g + r) * 16);
        it.d2 = *(const uint32_t *)(tb + 1024 + 4 * r);
    }
    template <int MV>
    __device__ static void block(const Item &it, const _Float16 *xrow, const _Float16 *, const float *Xrow,
                                 int ul, int g, const Lane &, f32x4 &acc) {
        const float d0 = h2f(it.d2), d1 = h2f(it.d2 >> 16);
        uint32_t magic = 0x64006400u;
        asm("" : "+v"(magic));
        const uint32_t w[4] = {it.q.x, it.q.y, it.q.z, it.q.w};
        f32x4 S[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            // bytes {0, 2} or {1, 3} of a word under the exponent byte 0x64 (byte 1 of magic,
            // selector 5): FP16 1024 + b with one v_perm_b32 per dword
            uint4 bq;
            bq.x = __builtin_amdgcn_perm(magic, w[2 * b], 0x05020500u);
            bq.y = __builtin_amdgcn_perm(magic, w[2 * b], 0x05030501u);
            bq.z = __builtin_amdgcn_perm(magic, w[2 * b + 1], 0x05020500u);
            bq.w = __builtin_amdgcn_perm(magic, w[2 * b + 1], 0x05030501u);
            // 1152 + q - 1152 = q, the signed quant, exact in FP16
            f16x8 bf = __builtin_bit_cast(f16x8, bq);
            bf = bf + f16x8{kOff, kOff, kOff, kOff, kOff, kOff, kOff, kOff};
            S[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8 *)(xrow + ul * 64 + 32 * b + 8 * g), bf,
                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MV; ++i) {
            acc[i] = __builtin_fmaf(d0, S[0][i], acc[i]);
            acc[i] = __builtin_fmaf(d1, S[1][i], acc[i]);
        }
    }
};

// Q6_K as a small-row format: item = one 256-element block of a 16-row tile. Step s (32 k,
// lane group g holding k = 32s + 8g + e) builds the FP16 operands 1024 + q6 from the low nibble
// and the two high bits, then q6 - 32 (quant.rs:43-61's signed quant) with one packed FP16
// subtraction of 1056, exact. The step's two 16-column scale groups (lane groups 0, 1: group
// 2s; groups 2, 3: group 2s + 1) come out of one MFMA for up to 8 rows (half_row), or of two
// MFMAs whose activations are masked to one half by a zero row. Then out += d sum_t sc_t S_t:
// the products x (q6 - 32) are exact, so no activation sums or bias terms are needed.
struct GQ6K {
    static constexpr _Float16 kQ6Off = (_Float16)-1056.0f;
    static constexpr int KU = 256;
    static constexpr int XG = 16;
    static constexpr bool kZeroRow = true;
    struct Item {
        uint4 a, b, c;
        uint32_t hv;  // scale bytes 4g .. 4g + 3 of row r
        uint32_t dv;  // FP16 d of row r
    };
    struct Lane {
        uint32_t sh;
    };
    __device__ static Lane lane_consts(int g) { return Lane{8u * (uint32_t)g}; }
    __device__ static void load(Item &it, const QmmParams &p, int tile, int u, int g, int r) {
        const uint8_t *tb = p.wq + ((size_t)tile * (size_t)(p.K / 256) + (size_t)u) * 3360u;
        const uint32_t lo = (uint32_t)(16 * g + r) * 16u;
        it.a = ld16(tb + lo);
        it.b = ld16(tb + 1024u + lo);
        it.c = ld16(tb + 2048u + lo);
        it.hv = *(const uint32_t *)(tb + 3072u + (uint32_t)(16 * r + 4 * g));
        it.dv = *(const uint16_t *)(tb + 3328u + (uint32_t)(2 * r));
    }
    template <int MV>
    __device__ static void block(const Item &it, const _Float16 *xrow, const _Float16 *xalt,
                                 const float *Xrow, int ul, int g, const Lane &c, f32x4 &acc) {
        const uint4 scw = q4k_head_gather(it.hv);  // the row's 16 scales, 4 per dword
        const uint32_t SC[4] = {scw.x, scw.y, scw.z, scw.w};
        const float d = h2f(it.dv);
        const uint32_t W[12] = {it.a.x, it.a.y, it.a.z, it.a.w, it.b.x, it.b.y,
                                it.b.z, it.b.w, it.c.x, it.c.y, it.c.z, it.c.w};
        uint32_t magic = 0x64006400u;
        asm("" : "+v"(magic));
        const int kb = ul * 256 + 8 * g;
        // MV <= 2: xalt is the lane's half_row pointer (both halves of a step in one MFMA);
        // MV = 4: xalt is the zero row, and each step runs an MFMA per half
        const _Float16 *xlo = (MV <= 2 ? xalt : (g < 2 ? xrow : xalt)) + kb;
        const _Float16 *xhi = (g < 2 ? xalt : xrow) + kb;
        float v[MV];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int hf = s >> 2, i = s & 3;
            const int qi = 2 * (2 * hf + (i & 1)), nib = 4 * (i >> 1);
            u32x4 bq;
#pragma unroll
            for (int p2 = 0; p2 < 2; ++p2) {
                // the four 6-bit values of one word, a byte each; v_perm_b32 then puts bytes
                // {0, 2} or {1, 3} under the exponent byte 0x64: FP16 1024 + q. Selector
                // bytes 0-3 pick bytes of q6, 5 picks byte 1 of magic (0x64).
                const uint32_t q6 = ((W[qi + p2] >> nib) & 0x0f0f0f0fu) |
                                    (((W[8 + 2 * hf + p2] >> (2 * i)) & 0x03030303u) << 4);
                bq[2 * p2] = __builtin_amdgcn_perm(magic, q6, 0x05020500u);
                bq[2 * p2 + 1] = __builtin_amdgcn_perm(magic, q6, 0x05030501u);
            }
            // 1024 + q6 - 1056 = q6 - 32, the signed quant, exact in FP16
            f16x8 bf = __builtin_bit_cast(f16x8, bq);
            bf = bf + f16x8{kQ6Off, kQ6Off, kQ6Off, kQ6Off, kQ6Off, kQ6Off, kQ6Off, kQ6Off};
            const int t0 = 2 * s, t1 = 2 * s + 1;
            const float sc0 = (float)(int32_t)(int8_t)((SC[t0 >> 2] >> (8 * (t0 & 3))) & 0xffu);
            const float sc1 = (float)(int32_t)(int8_t)((SC[t1 >> 2] >> (8 * (t1 & 3))) & 0xffu);
            if constexpr (MV <= 2) {
                // element 2a + h: accumulator row a, half h
                const f32x4 S = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8 *)(xlo + 32 * s), bf,
                                                                       f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int m = 0; m < MV; ++m) {
                    v[m] = s == 0 ? sc0 * S[2 * m] : __builtin_fmaf(sc0, S[2 * m], v[m]);
                    v[m] = __builtin_fmaf(sc1, S[2 * m + 1], v[m]);
                }
            } else {
                const f32x4 S0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8 *)(xlo + 32 * s), bf,
                                                                        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                const f32x4 S1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8 *)(xhi + 32 * s), bf,
                                                                        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int m = 0; m < MV; ++m) {
                    v[m] = s == 0 ? sc0 * S0[m] : __builtin_fmaf(sc0, S0[m], v[m]);
                    v[m] = __builtin_fmaf(sc1, S1[m], v[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MV; ++m) acc[m] = __builtin_fmaf(d, v[m], acc[m]);
    }
};

// Small-row kernel, one workgroup per TW consecutive 16-row tiles. Wave w of W owns items
// [w U / W, (w+1) U / W) (U = K / G::KU) of every tile of the workgroup: it issues its activation
// loads, then its first P (tile, item) loads, stages its own activation columns in a private LDS
// region (no workgroup barrier), and runs the items as they arrive, tile-major, refilling P
// items ahead when they do not all fit. A wave's partial sum of each tile goes to its own LDS
// region; after one barrier, wave t adds tile t's W partials in wave order. Each output element
// is the same sum for every M and TW. Many short workgroups keep every compute unit fed as the
// memory system serves them unevenly.
template <class G, int W, int TW, int P, int MV, int XB, bool GRP = false>
__device__ __forceinline__ void qmv_body(const QmmParams &p, int wt_off = 0) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int U = p.K / G::KU;
    const int T = p.N >> 4;
    const int tile0 = blockIdx.x * TW;
    const int ntw = min(TW, T - tile0);  // tiles of this workgroup (>= 1)
    const int u0 = wave * U / W;
    const int nu = (wave + 1) * U / W - u0;
    const int umax = (U + W - 1) / W;
    const int stride = umax * G::KU + kLdsPad;
    const int xstride = umax * (G::KU / G::XG);
    // per wave: FP16 activations [M][stride], sums [M][xstride], for formats that mask
    // activation fragments a zero row [stride], and the rows' range factors [M]; reused for the
    // partials
    const int zbytes = G::kZeroRow ? stride * 2 : 0;
    const int region = max((p.M * stride * 2 + p.M * xstride * 4 + zbytes + p.M * 4 + 15) & ~15, TW * 1024);
    uint8_t *mine = (uint8_t *)lds + (size_t)wave * region;
    _Float16 *xs = (_Float16 *)mine;
    float *Xs = (float *)(mine + p.M * stride * 2);
    _Float16 *zrow = (_Float16 *)(mine + p.M * stride * 2 + p.M * xstride * 4);
    float *Sc = (float *)(mine + p.M * stride * 2 + p.M * xstride * 4 + zbytes);
    const int nitems = nu * ntw;
    bool scaled = false;  // wave-uniform: this wave's rows carry range factors

    auto load_item = [&](typename G::Item &dst, int idx) {
        idx = min(idx, nitems - 1);
        const int tw = idx / nu;
        G::load(dst, p, wt_off + tile0 + tw, u0 + (idx - tw * nu), g, r16);
    };
    f32x4 acc[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nu > 0) {
        typename G::Item buf[P];
        auto issue = [&] {
#pragma unroll
            for (int j = 0; j < P; ++j) load_item(buf[j], j);
        };
        const int c0 = u0 * G::KU, nc = nu * G::KU;
        if (G::kZeroRow)
            for (int i = lane; i < stride / 8; i += 64) *(f16x8 *)(zrow + 8 * i) = f16x8{};
        if (p.act == 0)  // FP16 rows are in range by construction
            stage_wave_cols<0, XB, G::XG, GRP>(p, c0, nc, xs, stride, Xs, xstride, lane, issue);
        else if (p.act == 1)
            scaled = stage_wave_checked<1, XB, G::XG, GRP>(p, c0, nc, xs, stride, Xs, xstride, Sc, lane, issue);
        else
            scaled = stage_wave_checked<2, XB, G::XG, GRP>(p, c0, nc, xs, stride, Xs, xstride, Sc, lane, issue);
        // LDS operations of one wave complete in order; this keeps the compiler from moving
        // the fragment reads above the staging writes.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

        const int arow = spread_row(r16, (p.M + 3) >> 2, p.M);
        const _Float16 *xrow = xs + arow * stride;
        const float *Xrow = Xs + arow * xstride;
        const _Float16 *xalt = G::kZeroRow && MV <= 2 ? half_row(xs, zrow, stride, r16, g, p.M) : zrow;
        const typename G::Lane lc = G::lane_consts(g);
        for (int i0 = 0; i0 < nitems; i0 += P) {
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const int idx = i0 + j;
                if (idx < nitems) {
                    const int tw = idx / nu;
                    f32x4 a = acc[0];
#pragma unroll
                    for (int t = 1; t < TW; ++t)
                        if (t == tw) a = acc[t];
                    G::template block<MV>(buf[j], xrow, xalt, Xrow, idx - tw * nu, g, lc, a);
#pragma unroll
                    for (int t = 0; t < TW; ++t)
                        if (t == tw) acc[t] = a;
                }
                if (i0 + P < nitems) load_item(buf[j], idx + P);
            }
        }
    }
    if (scaled) {  // before the partials overwrite the factors
#pragma unroll
        for (int t = 0; t < TW; ++t) unscale_rows(acc[t], Sc, g, p.M);
    }
    // this wave's staging region is no longer read: it takes the partials
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    f32x4 *part = (f32x4 *)mine;
#pragma unroll
    for (int t = 0; t < TW; ++t) part[t * 64 + lane] = acc[t];
    lds_barrier();
    for (int t = wave; t < ntw; t += W) {
        f32x4 sum = ((const f32x4 *)lds)[t * 64 + lane];
        for (int w = 1; w < W; ++w) {
            const f32x4 v = ((const f32x4 *)((const uint8_t *)lds + (size_t)w * region))[t * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] += v[i];
        }
        const int col = (tile0 + t) * 16 + r16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = spread_out(g, i, (p.M + 3) >> 2, p.M);
            if (m >= 0) {
                const int mo = GRP ? (int)p.ids[m] : m;  // grouped: output row ids[s]
                const size_t o = (size_t)mo * (size_t)p.ldo + (size_t)col;
                if (p.out_type == 0)
                    ((float *)p.out)[o] = sum[i];
                else
                    ((uint16_t *)p.out)[o] = (uint16_t)f2bf(sum[i]);
            }
        }
    }
}

// Persistent variant of qmv_body for wide matrices (many more tiles than compute units):
// workgroup c owns tiles [c T / G, (c + 1) T / G) and stages its activation columns once. Each
// wave runs its (tile, item) list tile-major with P loads in flight across tile boundaries and
// writes its partial of every tile to an LDS slot; after every TS tiles one barrier, then wave t
// adds tile t's W partials in wave order (slots double-buffered, so the next chunk's partials
// never overwrite ones still being added). Every output element is the same sum as in qmv_body.
// GR: the greedy epilogue (FP32 outputs soft-capped, per-row partial argmax of the workgroup's
// columns; a variant of its own, so the plain kernels keep their registers).
template <class G, int W, int TS, int P, int MV, int XB, bool GR = false>
__device__ __forceinline__ void qmvp_body(const QmmParams &p) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int U = p.K / G::KU;
    const int T = p.N >> 4;
    const int t_begin = (int)((int64_t)blockIdx.x * T / gridDim.x);
    const int nt = (int)((int64_t)(blockIdx.x + 1) * T / gridDim.x) - t_begin;  // >= 1
    const int u0 = wave * U / W;
    const int nu = (wave + 1) * U / W - u0;
    const int umax = (U + W - 1) / W;
    const int stride = umax * G::KU + kLdsPad;
    const int xstride = umax * (G::KU / G::XG);
    const int zbytes = G::kZeroRow ? stride * 2 : 0;
    const int region = (p.M * stride * 2 + p.M * xstride * 4 + zbytes + p.M * 4 + 15) & ~15;  // bytes
    uint8_t *mine = (uint8_t *)lds + (size_t)wave * region;
    _Float16 *xs = (_Float16 *)mine;
    float *Xs = (float *)(mine + p.M * stride * 2);
    _Float16 *zrow = (_Float16 *)(mine + p.M * stride * 2 + p.M * xstride * 4);
    float *Sc = (float *)(mine + p.M * stride * 2 + p.M * xstride * 4 + zbytes);  // range factors
    f32x4 *part = (f32x4 *)((uint8_t *)lds + (size_t)W * region);  // [2][TS][W][64]
    bool scaled = false;  // wave-uniform: this wave's rows carry range factors

    int chunk = 0, tt = 0;
    Greedy gr[4] = {Greedy::none(), Greedy::none(), Greedy::none(), Greedy::none()};
    auto store = [&](int tile, const f32x4 &v) {
        const int col = tile * 16 + r16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = spread_out(g, i, (p.M + 3) >> 2, p.M);
            if (m >= 0) {
                const size_t o = (size_t)m * (size_t)p.ldo + (size_t)col;
                if constexpr (GR) {
                    const float c = soft_capped(v[i], p.cap);
                    ((float *)p.out)[o] = c;
                    if (i < MV) gr[i].add(c, col);  // rows per lane group <= MV
                } else if (p.out_type == 0) {
                    ((float *)p.out)[o] = v[i];
                } else {
                    ((uint16_t *)p.out)[o] = (uint16_t)f2bf(v[i]);
                }
            }
        }
    };
    // this wave's partial of tile tt of the current chunk is `a`
    auto end_tile = [&](const f32x4 &a) {
        const int tc = min(TS, nt - chunk * TS);
        f32x4 v = a;
        if (scaled) unscale_rows(v, Sc, g, p.M);
        part[(((chunk & 1) * TS + tt) * W + wave) * 64 + lane] = v;
        if (++tt == tc) {
            lds_barrier();
            for (int t = wave; t < tc; t += W) {
                const f32x4 *src = part + ((chunk & 1) * TS + t) * W * 64 + lane;
                f32x4 sum = src[0];
                for (int w = 1; w < W; ++w) {
                    const f32x4 v = src[w * 64];
#pragma unroll
                    for (int i = 0; i < 4; ++i) sum[i] += v[i];
                }
                store(t_begin + chunk * TS + t, sum);
            }
            ++chunk;
            tt = 0;
        }
    };

    // Staging and the first loads run at raised priority, so that a wave still staging goes
    // ahead of waves already at their arithmetic (m = 4 / 8 on the decode GEMV: 2 % faster; the
    // per-tile kernels were 1 % slower with it and keep the default).
    __builtin_amdgcn_s_setprio(3);
    if (nu > 0) {
        const int nitems = nu * nt;
        int ld_t = 0, ld_u = 0;  // (tile, item) of the next load
        auto load_next = [&](typename G::Item &dst) {
            G::load(dst, p, t_begin + ld_t, u0 + ld_u, g, r16);
            if (++ld_u == nu) {
                ld_u = 0;
                ld_t = min(ld_t + 1, nt - 1);  // past the end: reload the last tile (unused)
            }
        };
        typename G::Item buf[P];
        auto issue = [&] {
#pragma unroll
            for (int j = 0; j < P; ++j) load_next(buf[j]);
        };
        const int c0 = u0 * G::KU, nc = nu * G::KU;
        if (G::kZeroRow)
            for (int i = lane; i < stride / 8; i += 64) *(f16x8 *)(zrow + 8 * i) = f16x8{};
        if (p.act == 0)
            stage_wave_cols<0, XB, G::XG>(p, c0, nc, xs, stride, Xs, xstride, lane, issue);
        else if (p.act == 1)
            scaled = stage_wave_checked<1, XB, G::XG, false>(p, c0, nc, xs, stride, Xs, xstride, Sc, lane, issue);
        else
            scaled = stage_wave_checked<2, XB, G::XG, false>(p, c0, nc, xs, stride, Xs, xstride, Sc, lane, issue);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_setprio(0);

        const int arow = spread_row(r16, (p.M + 3) >> 2, p.M);
        const _Float16 *xrow = xs + arow * stride;
        const float *Xrow = Xs + arow * xstride;
        const _Float16 *xalt = G::kZeroRow && MV <= 2 ? half_row(xs, zrow, stride, r16, g, p.M) : zrow;
        const typename G::Lane lc = G::lane_consts(g);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        int ul = 0;
        for (int i0 = 0; i0 < nitems; i0 += P) {
#pragma unroll
            for (int j = 0; j < P; ++j) {
                if (i0 + j < nitems) {
                    G::template block<MV>(buf[j], xrow, xalt, Xrow, ul, g, lc, acc);
                    if (++ul == nu) {
                        end_tile(acc);
                        acc = f32x4{0.f, 0.f, 0.f, 0.f};
                        ul = 0;
                    }
                }
                if (i0 + P < nitems) load_next(buf[j]);
            }
        }
    } else {
        __builtin_amdgcn_s_setprio(0);
        for (int t = 0; t < nt; ++t) end_tile(f32x4{0.f, 0.f, 0.f, 0.f});
    }
    if constexpr (GR) {
        // per row, over the workgroup's columns: lane groups, then waves through the partial
        // slots of the chunk parity not read last (every wave finished reading them before
        // the last chunk's barrier)
        Greedy *red = (Greedy *)(part + (size_t)(chunk & 1) * TS * W * 64);  // [W][4 g][4 i]
#pragma unroll
        for (int i = 0; i < MV; ++i) gr[i].group16();
        if (r16 == 0) {
#pragma unroll
            for (int i = 0; i < MV; ++i) red[(wave * 4 + g) * 4 + i] = gr[i];
        }
        lds_barrier();
        if (wave == 0 && lane < p.M) {  // row `lane` is element i = lane % rpg of lane group lane / rpg
            const int rpg = (p.M + 3) >> 2, g2 = lane / rpg, i2 = lane - g2 * rpg;
            Greedy b = red[g2 * 4 + i2];
            for (int w = 1; w < W; ++w) b.merge(red[(w * 4 + g2) * 4 + i2]);
            b.fold(p.amax_key + lane, p.amax_bad + lane);
        }
    }
}

// Split-K variant of qmv_body: a workgroup of W waves owns W tiles and one of W K slices, slice
// s being the units [s U / W, (s + 1) U / W) that wave s covers in qmv_body. Its waves stage
// the slice's activation columns together, so each workgroup reads 1/W of the activations
// instead of all of them. Wave w computes tile w's partial over the slice (qmv_body's wave s
// chain for that tile), stores it to p.part and counts it on the tile's counter; the wave
// that completes the count adds the W partials in slice order and writes the outputs. That is qmv_body's sum, term for term, so every variant gives the same bits.
// Counters advance by 16 per launch (16 / W per wave) and so stay a multiple of 16 between
// launches for any W dividing 16. Block b maps to slice b / GP and tile group b % GP, GP =
// the group count rounded up to a multiple of 8, so that the slices of a group share an XCD.
template <class G, int W, int P, int MV, int XB>
__device__ __forceinline__ void qmvs_body(const QmmParams &p) {
    static_assert(16 % W == 0, "W must divide 16");
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int r16 = lane & 15;
    const int U = p.K / G::KU;
    const int T = p.N >> 4;
    const int groups = (T + W - 1) / W;
    const int gp = (groups + 7) & ~7;
    const int s = blockIdx.x / gp;
    const int tg = blockIdx.x - s * gp;
    if (tg >= groups) return;  // workgroup-uniform: padding of the XCD mapping
    const int u0 = s * U / W;
    const int nu = (s + 1) * U / W - u0;
    const int umax = (U + W - 1) / W;
    const int stride = umax * G::KU + kLdsPad;
    const int xstride = umax * (G::KU / G::XG);
    _Float16 *xs = (_Float16 *)lds;
    float *Xs = (float *)((uint8_t *)lds + p.M * stride * 2);
    _Float16 *zrow = (_Float16 *)((uint8_t *)lds + p.M * stride * 2 + p.M * xstride * 4);
    const int zbytes = G::kZeroRow ? stride * 2 : 0;
    float *Sc = (float *)((uint8_t *)lds + p.M * stride * 2 + p.M * xstride * 4 + zbytes);  // range factors
    int *wflag = (int *)(Sc + p.M);  // [W]: a wave's staging overflowed FP16
    bool scaled = false;             // workgroup-uniform
    const int tile = tg * W + wave;
    const bool live = tile < T;  // wave-uniform
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nu > 0) {  // workgroup-uniform
        typename G::Item buf[P];
        auto load_item = [&](typename G::Item &dst, int idx) {
            G::load(dst, p, tile, u0 + min(idx, nu - 1), g, r16);
        };
        auto issue = [&] {
            if (live) {
#pragma unroll
                for (int j = 0; j < P; ++j) load_item(buf[j], j);
            }
        };
        const int c0 = u0 * G::KU, nc = nu * G::KU;
        if (G::kZeroRow)
            for (int i = (int)threadIdx.x; i < stride / 8; i += 64 * W) *(f16x8 *)(zrow + 8 * i) = f16x8{};
        bool nf = false;
        if (p.act == 0)
            stage_group_cols<0, XB, G::XG, W>(p, c0, nc, xs, stride, Xs, xstride, lane, wave, issue);
        else if (p.act == 1)
            nf = stage_group_cols<1, XB, G::XG, W>(p, c0, nc, xs, stride, Xs, xstride, lane, wave, issue);
        else
            nf = stage_group_cols<2, XB, G::XG, W>(p, c0, nc, xs, stride, Xs, xstride, lane, wave, issue);
        if (lane == 0) wflag[wave] = __any(nf) ? 1 : 0;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
        for (int w = 0; w < W; ++w) scaled |= wflag[w] != 0;
        if (scaled) {  // some value overflowed FP16: the waves stage the slice again, row by row
            for (int r = wave; r < p.M; r += W) {
                if (p.act == 1)
                    stage_row_scaled<1, G::XG, false>(p, r, c0, nc, xs, stride, Xs, xstride, Sc, lane);
                else
                    stage_row_scaled<2, G::XG, false>(p, r, c0, nc, xs, stride, Xs, xstride, Sc, lane);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            lds_barrier();
        }
        if (live) {
            const int arow = spread_row(r16, (p.M + 3) >> 2, p.M);
            const _Float16 *xrow = xs + arow * stride;
            const float *Xrow = Xs + arow * xstride;
            const _Float16 *xalt = G::kZeroRow && MV <= 2 ? half_row(xs, zrow, stride, r16, g, p.M) : zrow;
            const typename G::Lane lc = G::lane_consts(g);
            for (int i0 = 0; i0 < nu; i0 += P) {
#pragma unroll
                for (int j = 0; j < P; ++j) {
                    const int idx = i0 + j;
                    if (idx < nu) G::template block<MV>(buf[j], xrow, xalt, Xrow, idx, g, lc, acc);
                    if (i0 + P < nu) load_item(buf[j], idx + P);
                }
            }
        }
    }
    if (!live) return;
    // the lane index again from mbcnt, so that it is not held in a register across the loop
    const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int lg = ln >> 4;
    const int col = tile * 16 + (ln & 15);
    const size_t plane = (size_t)p.M * (size_t)p.N;
    if (scaled) unscale_rows(acc, Sc, lg, p.M);
    // Partials are written and read as agent-scope atomics (sc1: through to the level every
    // compute unit sees, no cache-wide write-back or invalidate); the store acknowledgements are
    // awaited before the count, and the reads are issued only after the count completes. The
    // orderings are kept by the waits (hardware) and by asm memory clobbers (compiler), not by
    // release / acquire: an agent-scope fence on every wave (buffer_wbl2 sc1 + buffer_inv sc1, the
    // write-back and invalidation of the whole L2) made these kernels 4-17 times slower (Q4_K
    // 3840 x 15360 at M = 1: 190 against 11.4 us).
    const int rpg = (p.M + 3) >> 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = spread_out(lg, i, rpg, p.M);
        if (m >= 0)
            __hip_atomic_store(p.part + (size_t)s * plane + (size_t)m * p.N + col, acc[i],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint32_t old = 0;
    if (ln == 0)
        old = __hip_atomic_fetch_add(p.counters + tile, 16u / W, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (((old + 16u / W) & 15u) != 0) return;
    asm volatile("" ::: "memory");  // no partial read is moved above the count
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = spread_out(lg, i, rpg, p.M);
        if (m >= 0) {
            float sum = 0.f;
            for (int t = 0; t < W; ++t) {
                const float v = t == s ? acc[i]
                                       : __hip_atomic_load(p.part + (size_t)t * plane + (size_t)m * p.N + col,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sum = t == 0 ? v : sum + v;
            }
            const size_t o = (size_t)m * (size_t)p.ldo + (size_t)col;
            if (p.out_type == 0)
                ((float *)p.out)[o] = sum;
            else
                ((uint16_t *)p.out)[o] = (uint16_t)f2bf(sum);
        }
    }
}

}  // namespace

// One-tile workgroups run four per compute unit (8 waves per SIMD, at most 64 VGPRs); the
// library takes them for M <= 8, and two-tile workgroups (half the activation staging per weight
// byte) for larger M where the persistent kernel does not fit. MV = output rows kept per lane
// group (rows spread over the groups: M <= 4, M <= 8, M <= 16).
#define JV_QMV(TW, MV, XB)                                                                   \
    extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(TW == 1 ? 8 : 4))) \
    void jv_qmv_q4k_t##TW##_m##MV(QmmParams p) {                                             \
        qmv_body<GQ4K, 8, TW, 2 * TW, MV, XB>(p);                                            \
    }
JV_QMV(1, 1, 2)
JV_QMV(1, 2, 4)
JV_QMV(2, 4, 8)

// Q6_K: 8 waves, each two blocks of a tile at K = 3840 (all in flight); one tile per workgroup.
#define JV_QMV6(TW, MV, XB)                                                                  \
    extern "C" __global__ __launch_bounds__(512) void jv_qmv_q6k_t##TW##_m##MV(QmmParams p) { \
        qmv_body<GQ6K, 8, TW, 2 * TW, MV, XB>(p);                                            \
    }
JV_QMV6(1, 1, 2)
JV_QMV6(1, 2, 4)
JV_QMV6(1, 4, 8)

// Persistent kernels for wide matrices: chunks of two tiles, four items in flight per wave.
#define JV_QMVP(NAME, G, W, MV, XB)                                                          \
    extern "C" __global__ __launch_bounds__(64 * W) void jv_qmvp_##NAME##_m##MV(QmmParams p) { \
        qmvp_body<G, W, 2, 4, MV, XB>(p);                                                    \
    }                                                                                         \
    extern "C" __global__ __launch_bounds__(64 * W) void jv_qmvp_##NAME##_m##MV##_g(QmmParams p) { \
        qmvp_body<G, W, 2, 4, MV, XB, true>(p);                                              \
    }
// Activation loads in flight per lane (XB) cover the rows a variant stages: up to 4, 8 or 16.
JV_QMVP(q4k, GQ4K, 8, 1, 4)
JV_QMVP(q4k, GQ4K, 8, 2, 8)
JV_QMVP(q4k, GQ4K, 8, 4, 8)
JV_QMVP(q6k, GQ6K, 8, 1, 4)
JV_QMVP(q6k, GQ6K, 8, 2, 8)
JV_QMVP(q6k, GQ6K, 8, 4, 8)
JV_QMVP(q8_0, GQ8_0, 16, 1, 4)
JV_QMVP(q8_0, GQ8_0, 16, 2, 8)
JV_QMVP(q8_0, GQ8_0, 16, 4, 8)

// Q8_0: 16 waves, each four 64-k items of a tile at K = 4096 (all in flight).
#define JV_QMV8(TW, MV, XB)                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void jv_qmv_q8_0_t##TW##_m##MV(QmmParams p) { \
        qmv_body<GQ8_0, 16, TW, 4 * TW, MV, XB>(p);                                          \
    }
JV_QMV8(1, 1, 2)
JV_QMV8(1, 2, 4)
JV_QMV8(2, 4, 8)

// Expert-grouped small-row kernels (matvec_grouped, gemm.rs:1171-1203): grid y is the job, one
// 16-row weight tile of the job's expert per workgroup; the job's rows (at most rows_cap) are
// its sorted positions, read from input rows ids[s] / in_div and written to output rows
// ids[s]. Unused job slots return before any barrier. Jobs of up to 4 rows take the one-pass
// kernel _m1 (rows spread one per lane group), up to 8 rows _m2 (two per group). Larger jobs
// go through in chunks of 2 rows (_c2), a barrier between chunks (the next chunk's staging
// reuses the LDS the partials were read from), so the LDS holds 2 rows whatever rows_cap is;
// a later chunk reads the tile again, from L2. Every variant gives the same bits.
#define JV_QMVG_HEAD                                                                          \
    const int job = blockIdx.y;                                                               \
    if (job >= (int)p.jobs[0]) return;                                                        \
    const uint32_t e = p.jobs[1 + 2 * job];                                                   \
    const int js = (int)p.jobs[2 + 2 * job];                                                  \
    const int rows = min((int)(p.offsets[e + 1] - (uint32_t)js), p.rows_cap);
// jobs of at most MV rows (rows_cap <= MV): one pass
#define JV_QMVG(NAME, G, W, P, MV, XB)                                                        \
    extern "C" __global__ __launch_bounds__(64 * W) void jv_qmvg_##NAME##_m##MV(QmmParams p) { \
        JV_QMVG_HEAD                                                                          \
        QmmParams q = p;                                                                      \
        q.M = rows;                                                                           \
        q.ids = p.ids + js;                                                                   \
        qmv_body<G, W, 1, P, MV, XB, true>(q, (int)e * (p.N >> 4));                           \
    }
// jobs of more rows: chunks of 2 rows
#define JV_QMVGC(NAME, G, W, P)                                                               \
    extern "C" __global__ __launch_bounds__(64 * W) void jv_qmvg_##NAME##_c2(QmmParams p) {   \
        JV_QMVG_HEAD                                                                          \
        for (int r0 = 0; r0 < rows; r0 += 2) {                                                \
            if (r0 > 0) lds_barrier();                                                        \
            QmmParams q = p;                                                                  \
            q.M = min(2, rows - r0);                                                          \
            q.ids = p.ids + js + r0;                                                          \
            qmv_body<G, W, 1, P, 2, 4, true>(q, (int)e * (p.N >> 4));                         \
        }                                                                                     \
    }
// Q4_K on 4 waves of about three 256-k items each (8 waves: 8-22 % slower on 128 experts
// [1408, 2816] at 8 and 32 tokens x top-8)
JV_QMVG(q4k, GQ4K, 4, 3, 1, 2)
JV_QMVG(q4k, GQ4K, 4, 3, 2, 4)
JV_QMVGC(q4k, GQ4K, 4, 3)
// Q6_K and Q8_0 on 4 waves too (Q8_0 with 12 of its 64-k items in flight per wave). On the
// same expert shapes, the per-tile kernels' 8 waves (Q6_K) were 13-14 % slower; Q8_0's 16
// waves took 87 / 223 us and 8 waves 58 / 152 us against 48 / 119 us on 4 (8 / 32 tokens).
JV_QMVG(q6k, GQ6K, 4, 3, 1, 2)
JV_QMVG(q6k, GQ6K, 4, 3, 2, 4)
JV_QMVGC(q6k, GQ6K, 4, 3)
JV_QMVG(q8_0, GQ8_0, 4, 12, 1, 2)
JV_QMVG(q8_0, GQ8_0, 4, 12, 2, 4)
JV_QMVGC(q8_0, GQ8_0, 4, 12)

// Split-K kernels: W tiles x one K slice per workgroup (activation staging shared by the waves).
#define JV_QMVS(NAME, G, W, P, MV, XB, WPE)                                                  \
    extern "C" __global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE))) \
    void jv_qmvs_##NAME##_m##MV(QmmParams p) {                                               \
        qmvs_body<G, W, P, MV, XB>(p);                                                       \
    }
JV_QMVS(q4k, GQ4K, 8, 2, 1, 2, 8)
JV_QMVS(q4k, GQ4K, 8, 2, 2, 2, 8)
JV_QMVS(q4k, GQ4K, 8, 2, 4, 8, 4)
JV_QMVS(q6k, GQ6K, 8, 2, 1, 2, 4)
JV_QMVS(q6k, GQ6K, 8, 2, 2, 4, 4)
JV_QMVS(q6k, GQ6K, 8, 2, 4, 4, 3)
JV_QMVS(q8_0, GQ8_0, 16, 4, 1, 2, 4)
JV_QMVS(q8_0, GQ8_0, 16, 4, 2, 4, 4)
JV_QMVS(q8_0, GQ8_0, 16, 4, 4, 8, 4)

// ---------------------------------------------------------------------------------------------
// Entry points (looked up by name with hipModuleGetFunction).
// ---------------------------------------------------------------------------------------------
#define JV_QMM(NAME, F, MT, NT)                                                              \
    extern "C" __global__ __launch_bounds__(kThreads) void jv_qmm_##NAME##_m##MT##_n##NT(   \
        QmmParams p) {                                                                       \
        qmm_body<F, MT, NT>(p);                                                              \
    }
#define JV_QMM_TILES(NAME, F) \
    JV_QMM(NAME, F, 1, 1)     \
    JV_QMM(NAME, F, 1, 2)     \
    JV_QMM(NAME, F, 2, 1)     \
    JV_QMM(NAME, F, 2, 2)     \
    JV_QMM(NAME, F, 2, 4)     \
    JV_QMM(NAME, F, 4, 1)     \
    JV_QMM(NAME, F, 4, 2)     \
    JV_QMM(NAME, F, 4, 4)     \
    JV_QMM(NAME, F, 8, 1)     \
    JV_QMM(NAME, F, 8, 2)     \
    JV_QMM(NAME, F, 8, 4)

JV_QMM_TILES(q4k, FQ4K)
JV_QMM_TILES(q6k, FQ6K)
JV_QMM_TILES(q8_0, FQ8_0)
JV_QMM_TILES(q5_0, FQ5_0)
JV_QMM_TILES(f16, FF16)

#define JV_DEQ(NAME, F) \
    extern "C" __global__ __launch_bounds__(kThreads) void jv_dequant_##NAME(DequantParams p) { \
        dequant_body<F>(p);                                                                    \
    }
JV_DEQ(q4k, FQ4K)
JV_DEQ(q6k, FQ6K)
JV_DEQ(q8_0, FQ8_0)
JV_DEQ(q5_0, FQ5_0)
JV_DEQ(f16, FF16)

// Split-K combine: out[i] = sum_z part[z * len + i], z in increasing order (reduce_splits,
// gemm.rs:803-815), written as FP32 or BF16.
extern "C" __global__ __launch_bounds__(256) void jv_reduce_splits(const float *part, void *out,
                                                                   int64_t len, int splits,
                                                                   int out_type) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= len) return;
    float sum = 0.f;
    for (int z = 0; z < splits; ++z) sum += part[(int64_t)z * len + i];
    if (out_type == 0)
        ((float *)out)[i] = sum;
    else
        ((uint16_t *)out)[i] = (uint16_t)f2bf(sum);
}

// The 8 values at x[row][col .. col + 7] as raw words (one 16-byte load, two for FP32) ...
template <int ACT>
__device__ __forceinline__ void act8_load(const void *x, size_t o, u32x4 r[2]) {
    if (ACT == 2) {
        r[0] = *(const u32x4 *)((const float *)x + o);
        r[1] = *(const u32x4 *)((const float *)x + o + 4);
    } else {
        r[0] = *(const u32x4 *)((const uint16_t *)x + o);
    }
}
// ... multiplied by s (the inverse of the row's range factor, a power of two: exact) and rounded
// to nearest even into FP16; FP16 input is copied. Elements go through scalars (a bit cast of a
// vector element directly is miscompiled).
template <int ACT>
__device__ __forceinline__ f16x8 act8_cvt(const u32x4 r[2], float s) {
    if (ACT == 0) return __builtin_bit_cast(f16x8, r[0]);
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint32_t w;
        if (ACT == 2) {
            w = r[e >> 2][e & 3];
        } else {
            const uint32_t pair = r[0][e >> 1];
            w = (pair >> (16 * (e & 1))) << 16;
        }
        h[e] = (_Float16)(__builtin_bit_cast(float, w) * s);
    }
    return h;
}

// ---------------------------------------------------------------------------------------------
// Activation packing: rows -> FP16 MFMA A fragments (layout in qmm_params.h, PackXParams), or
// FP16 rows [M][K] (`rowmajor`, the generic tiled kernel's input).
//  - FP16 rows are copied (pack_copy: thread ((mt * U + u) * 2 + half) * 64 + lane moves
//    fragments s = 4 half .. 4 half + 3 of (mt, u), every store of a wave 1 KB contiguous).
//  - BF16 and FP32 rows (pack_rows: one wave per row and its whole K) are divided by their range
//    factor and rounded to nearest even. The factor is range_scale's: a power of two for rows
//    whose largest magnitude exceeds 16384 (crates/jevons-burn/src/kernels.rs:105, :120-130),
//    so the division is exact; 1 otherwise.
// rscale[R] receives each packed (or row-major) row's factor, for the product to multiply its
// outputs by; rows of padding and unused job slots are skipped.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ uint16_t *frag_dst(const PackXParams &p, int R, int c) {
    // chunk c (k = 8 c) of packed row R: fragment (mt U + u) 8 + s, lane 16 g + r
    if (p.rowmajor) return p.out + (size_t)R * (size_t)p.K + 8 * (size_t)c;
    const int U = p.K >> 8, mt = R >> 4, r16 = R & 15;
    const int u = c >> 5, s = (c >> 2) & 7, g = c & 3;
    return p.out + ((((size_t)mt * U + u) * 8 + s) * 64 + 16 * g + r16) * 8;
}

// Input row of packed row R (-1: padding or an unused row of a job; -2: an unused job slot).
__device__ __forceinline__ int packed_source(const PackXParams &p, int R) {
    if (!p.grouped) return R < p.M ? R : -1;
    const int per = p.rows_cap >> 4;
    const int job = (R >> 4) / per;
    if (job >= (int)p.jobs[0]) return -2;
    const int r = R - job * per * 16;
    const uint32_t e = p.jobs[1 + 2 * job], s0 = p.jobs[2 + 2 * job];
    return r < min((int)(p.offsets[e + 1] - s0), p.rows_cap) ? (int)(p.ids[s0 + r] / (uint32_t)p.in_div) : -1;
}

// BF16 / FP32 rows, P = p.rpw (1, 2 or 4) per workgroup of NW waves: thread t handles row t % P
// and its chunks t / P + (64 NW / P) i (8 values each), so a wave's store writes P consecutive
// rows' 16-byte pieces side by side for 64 / P chunks. The host picks P and NW so that each
// thread holds 8 chunks or fewer in registers between the row's maximum and its conversion, and
// small row counts still spread over many workgroups.
template <int ACT>
__device__ __forceinline__ void pack_rows(const PackXParams &p) {
    __shared__ float wmax[16][4];
    __shared__ int wnf[16][4];
    const int nthreads = (int)blockDim.x;  // 64 NW
    const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6;
    const int P = p.rpw;
    const int rr = t & (P - 1), cl = t / P, tpr = nthreads / P;  // row of the group, chunk lane, per row
    const int R = (int)blockIdx.x * P + rr;
    const int rows_out = p.rowmajor ? p.M : p.mtiles * 16;
    const int xr = R < rows_out ? packed_source(p, R) : -2;
    const int chunks = p.K >> 3;
    const size_t base = xr >= 0 ? (size_t)xr * (size_t)p.ldx : 0;
    constexpr int B = 8;  // chunks held per thread
    u32x4 r[B][2];
    // Loads past the row's end read its last chunk again (unused): unguarded loads stay in flight
    // together, where a branch around each would wait for the ones before it.
    auto load_batch = [&](int c0) {
#pragma unroll
        for (int j = 0; j < B; ++j)
            act8_load<ACT>(p.x, base + 8 * (size_t)min(c0 + tpr * j + cl, chunks - 1), r[j]);
    };
    float mx = 0.f;
    bool nf = false;
    const bool held = chunks <= tpr * B;  // one batch: the loads are kept for the conversion
    if (xr >= 0) {
        for (int c0 = 0; c0 < chunks; c0 += tpr * B) {
            load_batch(c0);
#pragma unroll
            for (int j = 0; j < B; ++j) {
                if (c0 + tpr * j + cl < chunks) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        uint32_t w;  // through a scalar: a bit cast of a vector element is miscompiled
                        if (ACT == 2) {
                            w = r[j][e >> 2][e & 3];
                        } else {
                            const uint32_t pair = r[j][0][e >> 1];
                            w = (pair >> (16 * (e & 1))) << 16;
                        }
                        const float v = __builtin_bit_cast(float, w);
                        nf |= !__builtin_isfinite(v);
                        mx = __builtin_fmaxf(mx, __builtin_fabsf(v));
                    }
                }
            }
        }
    }
    // the row's maximum over the lanes of its row (same t % P) and then over the waves
    int inf = nf ? 1 : 0;
    for (int off = P; off < 64; off <<= 1) {
        mx = __builtin_fmaxf(mx, __shfl_xor(mx, off));
        inf |= __shfl_xor(inf, off);
    }
    if (lane < P) {
        wmax[wave][rr] = mx;
        wnf[wave][rr] = inf;
    }
    __syncthreads();
    for (int w = 0; w < (nthreads >> 6); ++w) {
        mx = __builtin_fmaxf(mx, wmax[w][rr]);
        inf |= wnf[w][rr];
    }
    // Rows of padding (past M, or past a job's rows) and unused job slots are not written: the
    // products compute those rows from whatever the buffer holds and store none of them (an
    // output row depends on its own activation row only).
    if (xr < 0) return;
    float f;
    const float s = range_scale(inf ? __builtin_inff() : mx, &f);
    for (int c0 = 0; c0 < chunks; c0 += tpr * B) {
        if (!held) load_batch(c0);  // longer rows: read the batch again (from the cache)
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int c = c0 + tpr * j + cl;
            if (c < chunks) *(f16x8 *)frag_dst(p, R, c) = act8_cvt<ACT>(r[j], s);
        }
    }
    if (cl == 0) p.rscale[R] = f;
}

__device__ __forceinline__ void pack_copy(const PackXParams &p) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int U = p.K >> 8;
    if (t >= (int64_t)p.mtiles * U * 2 * 64) return;
    const int lane = (int)(t & 63);
    const int64_t q = t >> 6;
    const int half = (int)(q & 1);
    const int64_t mu = q >> 1;
    const int R = (int)(mu / U) * 16 + (lane & 15);  // packed row
    const int row = packed_source(p, R);
    if (row < 0) return;  // padding or an unused job slot: not written (pack_rows)
    const int col0 = (int)(mu % U) * 256 + half * 128 + (lane >> 4) * 8;
    uint16_t *dst = p.out + ((mu * 8 + 4 * half) * 64 + lane) * 8;
    u32x4 h[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
        h[s] = *(const u32x4 *)((const uint16_t *)p.x + (size_t)row * (size_t)p.ldx + (size_t)(col0 + 32 * s));
    if (mu % U == 0 && half == 0 && lane < 16) p.rscale[R] = 1.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) *(u32x4 *)(dst + s * 512) = h[s];
}

// Grid: FP16 fragments: mtiles * (K / 256) * 2 waves, 4 per workgroup; BF16 and FP32: one
// workgroup of 4 NW waves per 4 packed rows (rowmajor: rows). FP16 rows never take the
// row-major form.
extern "C" __global__ __launch_bounds__(1024) void jv_pack_x(PackXParams p) {
    if (p.act == 0)
        pack_copy(p);
    else if (p.act == 1)
        pack_rows<1>(p);
    else
        pack_rows<2>(p);
}

// ---------------------------------------------------------------------------------------------
// Pipelined tiled products (gemm_body below): weight fragments decoded once per workgroup into
// LDS, activation fragments from jv_pack_x's output, K in 32-k stages. Each output element is
// the same MFMA chain over K as in the other tiled kernels (32-k steps in order, lane group g
// holding k 32s + 8g .. +8), so the result is bitwise identical to theirs.
// ---------------------------------------------------------------------------------------------
namespace {


// All 8 (d s_j, dmin m_j) of row r of a block, from the lane's head dword (see q4k_item_load):
// lane group g decodes sub-blocks 2g, 2g + 1, and permlane swaps share them.
__device__ __forceinline__ void q4k_row_scales(uint32_t hv, int g, float dsc[8], float dmm[8]) {
    const uint4 hd = q4k_head_gather(hv);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    uint32_t sc[2], mn[2];
    q4k_pair_scales(hd, g, sc, mn);
    const uint4 a0 = q4k_head_gather(__builtin_bit_cast(uint32_t, d * (float)sc[0]));
    const uint4 a1 = q4k_head_gather(__builtin_bit_cast(uint32_t, d * (float)sc[1]));
    const uint4 b0 = q4k_head_gather(__builtin_bit_cast(uint32_t, dmin * (float)mn[0]));
    const uint4 b1 = q4k_head_gather(__builtin_bit_cast(uint32_t, dmin * (float)mn[1]));
    const uint32_t A0[4] = {a0.x, a0.y, a0.z, a0.w}, A1[4] = {a1.x, a1.y, a1.z, a1.w};
    const uint32_t B0[4] = {b0.x, b0.y, b0.z, b0.w}, B1[4] = {b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        dsc[2 * k] = __builtin_bit_cast(float, A0[k]);
        dsc[2 * k + 1] = __builtin_bit_cast(float, A1[k]);
        dmm[2 * k] = __builtin_bit_cast(float, B0[k]);
        dmm[2 * k + 1] = __builtin_bit_cast(float, B1[k]);
    }
}

// FP16 fragment of sub-block j for lane group g: elements 32j + 8g .. +7, decoded as
// quant.rs:25-41 does (low nibbles of byte pair j / 2 for even j, high nibbles for odd j).
__device__ __forceinline__ f16x8 q4k_sub_frag(const Q4KItem &it, int j, float dsc, float dmm) {
    const int pr = j >> 1;
    const uint32_t w0 = pr == 0 ? it.q0.x : pr == 1 ? it.q0.z : pr == 2 ? it.q1.x : it.q1.z;
    const uint32_t w1 = pr == 0 ? it.q0.y : pr == 1 ? it.q0.w : pr == 2 ? it.q1.y : it.q1.w;
    uint32_t n0 = (j & 1) ? (w0 >> 4) & 0x0f0f0f0fu : w0 & 0x0f0f0f0fu;
    uint32_t n1 = (j & 1) ? (w1 >> 4) & 0x0f0f0f0fu : w1 & 0x0f0f0f0fu;
    // Opaque to the compiler, so that each byte converts with one v_cvt_f32_ubyteN instead of a
    // bit-field extract of the known nibble plus a conversion.
    asm("" : "+v"(n0), "+v"(n1));
    // stored byte order {0, 2, 1, 3}: byte 1 holds element 2, byte 2 element 1
    const float q[8] = {(float)(uint8_t)n0, (float)(uint8_t)(n0 >> 16), (float)(uint8_t)(n0 >> 8),
                        (float)(uint8_t)(n0 >> 24), (float)(uint8_t)n1, (float)(uint8_t)(n1 >> 16),
                        (float)(uint8_t)(n1 >> 8), (float)(uint8_t)(n1 >> 24)};
    f16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f32_to_f16(__builtin_fmaf(q[e], dsc, -dmm));
    return v;
}

}  // namespace

// WM x WN waves; wave w = WN mq + nh computes m-tiles MT mq .. +MT and n-tiles NT nh .. +NT
// (MT = 16 / WM, NT = 8 / WN) of the 256 x 128 tile.
// Weight-fragment decoders of the tiled product. SPU = 32-k stages per K unit; load() reads the
// lane's raw bytes of weight row 16 tile + r for unit u, prep() its scales, frag() the FP16
// B fragment of stage s of the unit (lane (g, r): row r, k = 32 s + 8 g .. +8).
struct DQ4K {  // Q4_K: head dwords gathered across lane groups (q4k_row_scales)
    static constexpr int SPU = 8;
    static constexpr bool kDecodePrio = false;
    typedef Q4KItem Raw;
    struct Prep {
        float dsc[8], dmm[8];
    };
    __device__ static void load(Raw &it, const GemmParams &p, int tile, int u, int g, int r) {
        q4k_item_load(it, p.wq, p.K, tile, u, g, r);
    }
    __device__ static void prep(const Raw &it, Prep &pp, int g) { q4k_row_scales(it.hv, g, pp.dsc, pp.dmm); }
    __device__ static f16x8 frag(const Raw &it, const Prep &pp, int s, int) {
        return q4k_sub_frag(it, s, pp.dsc[s], pp.dmm[s]);
    }
};
template <class F>
struct DF {  // any format with the F* interface of the small-tile kernel
    static constexpr int SPU = F::KU / 32;
    // raised priority while decoding, on the 256 x 128 tile (measured there for Q6_K only)
    static constexpr bool kDecodePrio = std::is_same<F, FQ6K>::value;
    typedef typename F::Raw Raw;
    typedef typename F::Prep Prep;
    __device__ static void load(Raw &raw, const GemmParams &p, int tile, int u, int g, int r) {
        F::load(raw, p.wq, p.wh, p.wd, p.K, tile * 16 + r, u, g);
    }
    __device__ static void prep(const Raw &raw, Prep &pp, int g) { F::prep(raw, pp, g); }
    __device__ static f16x8 frag(const Raw &raw, const Prep &pp, int s, int g) { return frag_f16<F>(raw, pp, s, g); }
};

// Tiled product over packed activation fragments: a workgroup of WM x WN waves computes a
// (16 TM) x (16 TN) output tile; wave w = WN mq + nh computes m-tiles MT mq .. +MT and n-tiles
// NT nh .. +NT (MT = TM / WM, NT = TN / WN), MT x NT MFMA 16x16x32 accumulators. K advances
// in 32-k stages through four LDS buffers of (TM + TN) KB: per stage, wave w copies AS = TM / W
// activation fragments (1 KB each, lane order) from jv_pack_x's output and decodes BS = TN / W
// weight fragments (D::frag, the reference's FP16 tile format), so every weight is decoded once
// per workgroup. A wave takes the fragments it wrote from its registers and reads the others
// from LDS; the reads for stage t + 1 are issued while stage t's MFMAs run, and stage t + 2 is
// written meanwhile. Raw weights are loaded 8 stages ahead. Register slots are ordered
// own-first, so which fragment is whose is fixed at compile time. Requires K % 256 == 0.
// Split-K (grid z, ungrouped): slice z runs the same pipeline over its own K units, the generic
// kernel's slice z (whole 256-element blocks), from a zero accumulator, and writes its FP32
// partial for jv_reduce_splits; so a split plan gives the generic kernel's bits.
//
// Each output element is the same MFMA chain over K as in the other tiled kernels (32-k steps
// in order, lane group g holding k 32s + 8g .. +8), so the result is bitwise identical to theirs.
// GR: the greedy epilogue (FP32 outputs soft-capped, per-row partial argmax of the tile's
// columns; a variant of its own).
template <class D, int TM, int TN, int WM, int WN, bool HB = false, bool APRIV = false, int NVS = 3,
          bool GR = false>
__device__ __forceinline__ void gemm_body(const GemmParams &p) {
    constexpr int W = WM * WN, MT = TM / WM, NT = TN / WN;
    // activation fragments a wave loads per stage (own m slots): a share of its MT, or with
    // APRIV all of them (waves of one row of the wave grid load the same ones)
    constexpr int AS = APRIV ? MT : MT / WN;
    constexpr int BS = NT / WM;  // weight fragments a wave decodes per stage (own n slots)
    constexpr int UPS = 8 / D::SPU;  // K units per 8 stages
    // Activation fragments go through LDS only when several waves share an m-tile (WN > 1);
    // with WN = 1 every wave loads all of its own fragments and LDS holds only the weights.
    constexpr bool ASH = AS < MT;
    constexpr int AOFF = ASH ? TM * 1024 : 0;  // weight fragments' offset in a buffer
    constexpr int BUF = AOFF + TN * 1024;
    static_assert((APRIV || AS * W == TM) && BS * W == TN && AS >= 1 && BS >= 1, "tile split");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int mq = w / WN, nh = w % WN;
    // this slice's K units (the whole K without split-K), in blocks of 8 stages
    const int U_all = (p.K >> 5) / D::SPU;
    const int uf = (int)((int64_t)blockIdx.z * U_all / p.splits);
    const int zb0 = uf / UPS;                                                         // first block
    const int U8 = ((int)((int64_t)(blockIdx.z + 1) * U_all / p.splits) - uf) / UPS;  // blocks
    const int UK = U8 * UPS;          // K units
    const int mt0 = blockIdx.y * TM;  // first 16-row activation tile
    const int t0 = blockIdx.x * TN;   // first 16-row weight tile
    // expert-grouped: job blockIdx.y, its expert's weight tiles, rows, first sorted position
    int wt0 = 0, rows_real = 0, js = 0;
    if (p.grouped) {
        const int job = blockIdx.y;
        if (job >= (int)p.jobs[0]) return;  // workgroup-uniform, before any barrier
        const uint32_t e = p.jobs[1 + 2 * job];
        js = (int)p.jobs[2 + 2 * job];
        rows_real = min((int)(p.offsets[e + 1] - (uint32_t)js), p.rows_cap);
        wt0 = (int)e * (p.N >> 4);
    }
    const int stages = 8 * U8;
    const size_t stot = (size_t)(p.K >> 5);  // stages of the whole K
    const uint32_t lo16 = (uint32_t)lane * 16u;  // this lane's bytes in a 1 KB fragment

    // Local m-tile of slot i: own slots first (the AS this wave stages), then the rest of the
    // wave's MT in order; n-tile of slot k likewise with the BS tiles it decodes.
    auto m_of = [&](int i) __attribute__((always_inline)) {
        const int own0 = APRIV ? 0 : AS * nh;
        return MT * mq + (i < AS ? own0 + i : ((own0 + i) % MT));
    };
    auto n_of = [&](int k) __attribute__((always_inline)) {
        const int own0 = BS * mq;
        return NT * nh + (k < BS ? own0 + k : ((own0 + k) % NT));
    };

    // The packed fragment of m-tile mt at stage st is fragment mt (K / 32) + st: consecutive
    // stages of one m-tile are consecutive 1 KB fragments.
    const uint8_t *xa_own[AS];
#pragma unroll
    for (int i = 0; i < AS; ++i)
        xa_own[i] = (const uint8_t *)p.xa + ((size_t)(mt0 + m_of(i)) * stot + 8 * (size_t)zb0) * 1024u + lo16;
    auto load_a = [&](u32x4 *dst, int st) __attribute__((always_inline)) {
        const uint32_t off = (uint32_t)min(st, stages - 1) * 1024u;
#pragma unroll
        for (int i = 0; i < AS; ++i) dst[i] = *(const u32x4 *)(xa_own[i] + off);
    };
    // four LDS buffers, stage st in buffer st % 4 (a compile-time index in the unrolled loop)
    auto buf_of = [&](int st) __attribute__((always_inline)) { return smem + (st & 3) * BUF + lo16; };
    auto store_a = [&](const u32x4 *src, int st) __attribute__((always_inline)) {
        if constexpr (ASH) {
            uint8_t *base = buf_of(st);
#pragma unroll
            for (int i = 0; i < AS; ++i) *(u32x4 *)(base + m_of(i) * 1024) = src[i];
        }
    };
    // raw weights of the 8 stages from stage 8 b on (K units UPS b .. UPS b + UPS - 1)
    auto load_w = [&](typename D::Raw (*dst)[BS], int b) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < UPS; ++q)
#pragma unroll
            for (int k = 0; k < BS; ++k)
                D::load(dst[q][k], p, wt0 + t0 + n_of(k), UPS * zb0 + min(UPS * b + q, UK - 1), g, r);
    };
    typename D::Prep pp[UPS][BS];
    auto block_prep = [&](const typename D::Raw (*it)[BS]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < UPS; ++q)
#pragma unroll
            for (int k = 0; k < BS; ++k) D::prep(it[q][k], pp[q][k], g);
    };
    auto store_b = [&](const f16x8 *v, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < BS; ++k) *(f16x8 *)(buf_of(st) + AOFF + n_of(k) * 1024) = v[k];
    };
    // the fragments of stage st this wave does not hold
    auto read_other = [&](f16x8 *fa, f16x8 *fb, int st) __attribute__((always_inline)) {
        const uint8_t *base = buf_of(st);
#pragma unroll
        for (int i = 0; i < MT - AS; ++i) fa[i] = *(const f16x8 *)(base + m_of(AS + i) * 1024);
#pragma unroll
        for (int k = 0; k < NT - BS; ++k) fb[k] = *(const f16x8 *)(base + AOFF + n_of(BS + k) * 1024);
    };

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int k = 0; k < NT; ++k) acc[i][k] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto mfma_stage = [&](const u32x4 *aown, const f16x8 *bown, const f16x8 *fa, const f16x8 *fb)
        __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const f16x8 a = i < AS ? __builtin_bit_cast(f16x8, aown[i]) : fa[i - AS];
#pragma unroll
            for (int k = 0; k < NT; ++k)
                acc[i][k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, k < BS ? bown[k] : fb[k - BS], acc[i][k], 0, 0, 0);
        }
    };
    auto decode = [&](f16x8 *dst, const typename D::Raw (*it)[BS], int j) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < BS; ++k) dst[k] = D::frag(it[j / D::SPU][k], pp[j / D::SPU][k], j % D::SPU, g);
    };

    // Register sets: own activation fragments of stages t .. t + 3 (index t % 4), own decoded
    // weight fragments of stages t .. t + LEAD (index t % 4), other fragments read from LDS for
    // stages t, t + 1 (index t % 2).
    typename D::Raw cur[UPS][BS], nxt[UPS][BS];
    u32x4 A[4][AS];
    f16x8 B[4][BS];
    f16x8 FA[2][MT - AS > 0 ? MT - AS : 1], FB[2][NT - BS > 0 ? NT - BS : 1];
    load_w(cur, 0);
    load_w(nxt, 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) load_a(A[t], t);
    block_prep(cur);
    // Stages are written LEAD ahead of their MFMAs: 2, with a barrier after every stage, or,
    // with HB (only weights in LDS), 3 with a barrier after every odd stage. Then a buffer
    // written at step t is read at step t + 2 and rewritten at step t + 4, and every such pair
    // of steps straddles an odd step's barrier. The one exception is stage 0, read after the
    // prologue's barrier and rewritten (as stage 4) at step 1: with HB a second barrier follows
    // that read (each wave's fence waits for its own read to complete first).
    static_assert(!HB || !ASH, "half barriers need activation fragments in registers");
    constexpr int LEAD = HB ? 3 : 2;
#pragma unroll
    for (int t = 0; t < LEAD; ++t) {
        decode(B[t], cur, t);
        store_b(B[t], t);
        store_a(A[t], t);
    }
    lds_barrier();
    read_other(FA[0], FB[0], 0);
    if constexpr (HB) lds_barrier();

    // Stage st (j = st % 8): read stage st + 1's other fragments, MFMAs of stage st, write
    // stage st + LEAD (decode its weight fragments, store its activation fragments), then load
    // stage st + 4's activations into the registers stage st used. `tail` guards the stages
    // near the end of K; the other stages are branch-free, and their instructions are
    // interleaved so the decode, LDS traffic and loads issue between the MFMAs.
    auto step = [&](int st, int j, bool tail) __attribute__((always_inline)) {
        const int c = j & 3, f = j & 1;
        const int j2 = (j + LEAD) & 7;
        if (!tail || st + 1 < stages) read_other(FA[f ^ 1], FB[f ^ 1], st + 1);
        if (!tail || st + LEAD < stages) {
            if (j2 == 0) {  // stage st + LEAD starts a block of 8: its raw weights are in nxt
#pragma unroll
                for (int q = 0; q < UPS; ++q)
#pragma unroll
                    for (int k = 0; k < BS; ++k) cur[q][k] = nxt[q][k];
                load_w(nxt, (st + LEAD) / 8 + 1);
                block_prep(cur);
            }
            // Q6_K 256 x 128: the wave decoding its weight fragments runs at raised priority
            // (the down projection split eight ways: 4 % faster; Q4_K's tile 1 % slower)
            if constexpr (TM == 16 && D::kDecodePrio) __builtin_amdgcn_s_setprio(3);
            decode(B[(c + LEAD) & 3], cur, j2);
            store_b(B[(c + LEAD) & 3], st + LEAD);
            store_a(A[(c + LEAD) & 3], st + LEAD);
            if constexpr (TM == 16 && D::kDecodePrio) __builtin_amdgcn_s_setprio(0);
        }
        // The wave issuing its stage's MFMAs runs at raised priority, so that of the three or
        // four waves per SIMD the 32 x 64 and 128 x 128 tiles hold, the one at its MFMAs issues
        // them ahead of the others' decode and loads (7-9 % faster; the 256 x 128 tile, at two
        // waves per SIMD, did not change, and keeps the default).
        if constexpr (TM < 16) __builtin_amdgcn_s_setprio(3);
        mfma_stage(A[c], B[c], FA[f], FB[f]);
        if constexpr (TM < 16) __builtin_amdgcn_s_setprio(0);
        load_a(A[c], st + 4);
        if (!tail && j2 != 0) {
            constexpr int NM = MT * NT;                       // MFMAs of the stage
            constexpr int NR = (MT - AS) + (NT - BS);         // LDS reads
            constexpr int NW = (ASH ? AS : 0) + BS;           // LDS writes
            constexpr int NV = NVS;                           // VALU per MFMA slot
#pragma unroll
            for (int i = 0; i < NM; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, NV, 0); // VALU
                if (i < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                            // DS read
                else if (i >= NM / 2 && i < NM / 2 + NW) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
                else if (i >= NM - AS - 2 && i < NM - 2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // VMEM read
            }
        }
        if (!HB || (j & 1)) lds_barrier();
    };
    for (int b = 0; b + 1 < U8; ++b) {
#pragma unroll
        for (int j = 0; j < 8; ++j) step(8 * b + j, j, false);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) step(8 * (U8 - 1) + j, j, true);

    // epilogue: lane (g, r) holds column r, rows 4g .. 4g + 3 of each 16 x 16 tile
    const bool f32_out = p.out_type == 0;
    Greedy gr[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) gr[i][e] = Greedy::none();
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            const int col = (t0 + n_of(k)) * 16 + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pr = (mt0 + m_of(i)) * 16 + 4 * g + e;  // packed row
                int m = pr;
                bool live = m < p.M;
                if (p.grouped) {
                    const int ml = m_of(i) * 16 + 4 * g + e;  // row within the job
                    live = ml < rows_real;
                    if (live) m = (int)p.ids[js + ml];
                }
                if (live) {
                    const size_t o = (size_t)m * (size_t)p.ldo + (size_t)col;
                    const float v = acc[i][k][e] * p.rscale[pr];  // exact: a power of two
                    if constexpr (GR) {  // ungrouped, whole K, FP32 outputs (the host's rule)
                        // kept in place and stored after the count (below)
                        const float c = soft_capped(v, p.cap);
                        acc[i][k][e] = c;
                        gr[i][e].add(c, col);
                    } else if (p.splits > 1) {
                        p.part[(int64_t)blockIdx.z * p.split_stride + (int64_t)o] = v;
                    } else if (f32_out) {
                        ((float *)p.out)[o] = v;
                    } else {
                        ((uint16_t *)p.out)[o] = (uint16_t)f2bf(v);
                    }
                }
            }
        }
    }
    if constexpr (GR) {
        // per row over the tile's columns: the 16 lanes of a group, then the WN waves that
        // share the row, through the LDS buffers (every wave is past its last stage's reads
        // after the first barrier)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) gr[i][e].group16();
        lds_barrier();
        Greedy *red = (Greedy *)smem;  // [16 TM rows][WN]
        if (r == 0) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[(m_of(i) * 16 + 4 * g + e) * WN + nh] = gr[i][e];
        }
        lds_barrier();
        for (int t = (int)threadIdx.x; t < 16 * TM; t += 64 * W) {
            const int pr = mt0 * 16 + t;
            if (pr < p.M) {
                Greedy b = red[t * WN];
#pragma unroll
                for (int c = 1; c < WN; ++c) b.merge(red[t * WN + c]);
                b.fold(p.amax_key + pr, p.amax_bad + pr);
            }
        }
        // no wait: the keys are read by jv_greedy_finish after the launch
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int k = 0; k < NT; ++k) {
                const int col = (t0 + n_of(k)) * 16 + r;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = (mt0 + m_of(i)) * 16 + 4 * g + e;
                    if (m < p.M) ((float *)p.out)[(size_t)m * (size_t)p.ldo + (size_t)col] = acc[i][k][e];
                }
            }
        }
    }
}

// 64 x 64 tile on 8 waves, two per SIMD: wave w computes m-tile w / 2 against n-tiles 2 (w % 2)
// and 2 (w % 2) + 1 (two MFMAs a stage) with its activation fragments in registers, and wave
// 4 p + q decodes n-tile q's weight fragment of the stages of parity p, so every fragment is
// still decoded once per workgroup. The stages go through the same four LDS buffers as in
// gemm_body's HB tiles: written three stages ahead, a barrier after every odd step and one
// after the prologue's read of stage 0, so a buffer written at step t is read at step t + 2 and
// rewritten at step t + 4 with a barrier between each pair. Each output element is gemm_body's
// MFMA chain, so the bits are the same. Two waves per SIMD where the 4-wave tile runs one:
// down projection 89 against 97 us, q/k/v/o 10-14 % faster. Ungrouped products only: expert
// jobs (thousands of workgroups, already several per CU) ran slower on it (169 against 149 us
// on 128 experts x 32 rows).
// GR: the greedy epilogue, as in gemm_body.
template <class D, bool GR = false>
__device__ __forceinline__ void gemm8_body(const GemmParams &p) {
    constexpr int UPS = 8 / D::SPU;
    constexpr int LEAD = 3;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int mq = w >> 1, nh = w & 1;   // compute: m-tile mq, n-tiles 2 nh and 2 nh + 1
    const int par = w >> 2, dq = w & 3;  // decode: n-tile dq of the stages of parity par
    // this slice's K units (the whole K without split-K), in blocks of 8 stages
    const int U_all = (p.K >> 5) / D::SPU;
    const int uf = (int)((int64_t)blockIdx.z * U_all / p.splits);
    const int zb0 = uf / UPS;
    const int U8 = ((int)((int64_t)(blockIdx.z + 1) * U_all / p.splits) - uf) / UPS;
    const int UK = U8 * UPS;
    const int stages = 8 * U8;
    const int mt0 = blockIdx.y * 4, t0 = blockIdx.x * 4;
    const uint32_t lo16 = (uint32_t)lane * 16u;
    const uint8_t *xa = (const uint8_t *)p.xa +
                        ((size_t)(mt0 + mq) * (size_t)(p.K >> 5) + 8 * (size_t)zb0) * 1024u + lo16;
    auto load_a = [&](u32x4 &dst, int st) __attribute__((always_inline)) {
        dst = *(const u32x4 *)(xa + (uint32_t)min(st, stages - 1) * 1024u);
    };
    auto buf_of = [&](int st) __attribute__((always_inline)) { return smem + (st & 3) * 4096 + lo16; };
    auto load_w = [&](typename D::Raw *dst, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < UPS; ++q) D::load(dst[q], p, t0 + dq, UPS * zb0 + min(UPS * b + q, UK - 1), g, r);
    };
    typename D::Prep pp[UPS];
    auto block_prep = [&](const typename D::Raw *it) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < UPS; ++q) D::prep(it[q], pp[q], g);
    };
    auto read_b = [&](f16x8 *fb, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 2; ++k) fb[k] = *(const f16x8 *)(buf_of(st) + (2 * nh + k) * 1024);
    };
    typename D::Raw cur[UPS], nxt[UPS];
    u32x4 A[4];
    f16x8 FB[2][2];
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    load_w(cur, 0);
    load_w(nxt, 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) load_a(A[t], t);
    block_prep(cur);
#pragma unroll
    for (int t = 0; t < LEAD; ++t)
        if ((t & 1) == par)
            *(f16x8 *)(buf_of(t) + dq * 1024) = D::frag(cur[t / D::SPU], pp[t / D::SPU], t % D::SPU, g);
    lds_barrier();
    read_b(FB[0], 0);
    lds_barrier();

    auto step = [&](int st, int j, bool tail) __attribute__((always_inline)) {
        const int c = j & 3, f = j & 1;
        const int j2 = (j + LEAD) & 7;
        if (!tail || st + 1 < stages) read_b(FB[f ^ 1], st + 1);
        if (!tail || st + LEAD < stages) {
            if (j2 == 0) {  // stage st + LEAD starts a block of 8: its raw weights are in nxt
#pragma unroll
                for (int q = 0; q < UPS; ++q) cur[q] = nxt[q];
                load_w(nxt, (st + LEAD) / 8 + 1);
                block_prep(cur);
            }
            if ((j2 & 1) == par)
                *(f16x8 *)(buf_of(st + LEAD) + dq * 1024) =
                    D::frag(cur[j2 / D::SPU], pp[j2 / D::SPU], j2 % D::SPU, g);
        }
        const f16x8 a = __builtin_bit_cast(f16x8, A[c]);
#pragma unroll
        for (int k = 0; k < 2; ++k) acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, FB[f][k], acc[k], 0, 0, 0);
        load_a(A[c], st + 4);
        if (j & 1) lds_barrier();
    };
    for (int b = 0; b + 1 < U8; ++b) {
#pragma unroll
        for (int j = 0; j < 8; ++j) step(8 * b + j, j, false);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) step(8 * (U8 - 1) + j, j, true);

    const bool f32_out = p.out_type == 0;
    Greedy gr[4] = {Greedy::none(), Greedy::none(), Greedy::none(), Greedy::none()};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int col = (t0 + 2 * nh + k) * 16 + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = (mt0 + mq) * 16 + 4 * g + e;
            if (m < p.M) {
                const size_t o = (size_t)m * (size_t)p.ldo + (size_t)col;
                const float v = acc[k][e] * p.rscale[m];  // exact: a power of two
                if constexpr (GR) {  // ungrouped, whole K, FP32 outputs (the host's rule)
                    // kept in place and stored after the count (below)
                    const float c = soft_capped(v, p.cap);
                    acc[k][e] = c;
                    gr[e].add(c, col);
                } else if (p.splits > 1) {
                    p.part[(int64_t)blockIdx.z * p.split_stride + (int64_t)o] = v;
                } else if (f32_out) {
                    ((float *)p.out)[o] = v;
                } else {
                    ((uint16_t *)p.out)[o] = (uint16_t)f2bf(v);
                }
            }
        }
    }
    if constexpr (GR) {
        // per row over the tile's 64 columns: the 16 lanes of a group, then the two waves
        // (nh = 0, 1) of the m-tile through the stage buffers, after a barrier
#pragma unroll
        for (int e = 0; e < 4; ++e) gr[e].group16();
        lds_barrier();
        Greedy *red = (Greedy *)smem;  // [64 rows][2]
        if (r == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) red[(mq * 16 + 4 * g + e) * 2 + nh] = gr[e];
        }
        lds_barrier();
        const int t = (int)threadIdx.x, pr = mt0 * 16 + t;
        if (t < 64 && pr < p.M) {
            Greedy b = red[2 * t];
            b.merge(red[2 * t + 1]);
            b.fold(p.amax_key + pr, p.amax_bad + pr);
        }
        // no wait: the keys are read by jv_greedy_finish after the launch
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int col = (t0 + 2 * nh + k) * 16 + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = (mt0 + mq) * 16 + 4 * g + e;
                if (m < p.M) ((float *)p.out)[(size_t)m * (size_t)p.ldo + (size_t)col] = acc[k][e];
            }
        }
    }
}

// Tiles (rows x columns): 256 x 128 and 128 x 128 on 8 waves of 4 x 2, 64 x 64 on 4 waves of
// 2 x 2, activation fragments shared through LDS. Q4_K, Q6_K and Q8_0 also have all three tiles
// with suffix r, whose waves keep their activation fragments in registers, so LDS holds only
// the weights, writing stages three ahead with a barrier every second stage (HB): Q4_K and Q6_K
// 256 x 128 on 8 waves of 8 x 1 (32 x 128 each); Q8_0 256 x 128 and every 128 x 128 and 64 x 64
// on the 4 x 2 / 2 x 2 grid with each wave loading all of its m-tiles (APRIV, waves of one grid
// row load the same fragments) and reading only its share of the weights from LDS. These three
// formats also have a 32 x 64 r tile (2 x 2 waves of 16 x 32) for products of up to 32 rows,
// which a 64-row tile would half fill, and a 32 x 128 r tile (2 x 2 waves of 16 x 64) for the
// 32 x 128 plans (slower than 32 x 64, which the library's own plans take; faster than the
// generic tiles that ran those plans).
// Those are the library's tiles for these formats (the faster arrangement per format and tile
// in interleaved measurements); the same bits either way. The last argument is how many VALU
// instructions the scheduler places after each MFMA of a stage (the weight decode is spread
// over the MFMAs): 4 for Q4_K and 5 for Q6_K on 256 x 128 (2 x 8 MFMAs per stage), 1 for the
// Q4_K 64 x 64 and the Q4_K / Q6_K 128 x 128 tiles, 2 for 32 x 64, 3 elsewhere, each the
// fastest of 1 .. 5 (1 .. 3 for 32 x 64) in interleaved measurements (3 to 9 % over 3 where it
// differs).
#define JV_GEMM(NAME, D, TM, TN, WM, WN, ROWS, COLS, SUF, HB, NV)                             \
    extern "C" __global__ __launch_bounds__(64 * WM * WN) void jv_gemm_##NAME##_##ROWS##x##COLS##SUF(GemmParams p) { \
        gemm_body<D, TM, TN, WM, WN, HB, false, NV>(p);                                       \
    }
#define JV_GEMMP(NAME, D, TM, TN, WM, WN, ROWS, COLS, SUF, NV)                                \
    extern "C" __global__ __launch_bounds__(64 * WM * WN) void jv_gemm_##NAME##_##ROWS##x##COLS##SUF(GemmParams p) { \
        gemm_body<D, TM, TN, WM, WN, true, true, NV>(p);                                      \
    }
#define JV_GEMM_TILES(NAME, D)                                                                \
    JV_GEMM(NAME, D, 16, 8, 4, 2, 256, 128, , false, 3) JV_GEMM(NAME, D, 8, 8, 4, 2, 128, 128, , false, 3) \
    JV_GEMM(NAME, D, 4, 4, 2, 2, 64, 64, , false, 3)
JV_GEMM(q4k, DQ4K, 16, 8, 8, 1, 256, 128, r, true, 4)
JV_GEMM(q6k, DF<FQ6K>, 16, 8, 8, 1, 256, 128, r, true, 5)
JV_GEMMP(q8_0, DF<FQ8_0>, 16, 8, 4, 2, 256, 128, r, 3)
JV_GEMMP(q4k, DQ4K, 4, 4, 2, 2, 64, 64, r, 1)
JV_GEMMP(q6k, DF<FQ6K>, 4, 4, 2, 2, 64, 64, r, 3)
JV_GEMMP(q8_0, DF<FQ8_0>, 4, 4, 2, 2, 64, 64, r, 3)
JV_GEMMP(q4k, DQ4K, 8, 8, 4, 2, 128, 128, r, 1)
JV_GEMMP(q6k, DF<FQ6K>, 8, 8, 4, 2, 128, 128, r, 1)
JV_GEMMP(q8_0, DF<FQ8_0>, 8, 8, 4, 2, 128, 128, r, 3)
JV_GEMMP(q4k, DQ4K, 2, 4, 2, 2, 32, 64, r, 2)
JV_GEMMP(q6k, DF<FQ6K>, 2, 4, 2, 2, 32, 64, r, 2)
JV_GEMMP(q8_0, DF<FQ8_0Mix>, 2, 4, 2, 2, 32, 64, r, 2)
JV_GEMMP(q4k, DQ4K, 2, 8, 2, 2, 32, 128, r, 2)
JV_GEMMP(q6k, DF<FQ6K>, 2, 8, 2, 2, 32, 128, r, 2)
JV_GEMMP(q8_0, DF<FQ8_0Mix>, 2, 8, 2, 2, 32, 128, r, 2)
// The register tiles above with the greedy epilogue (vocabulary projections): the same
// template arguments and a _g suffix.
#define JV_GEMMG(NAME, D, TM, TN, WM, WN, ROWS, COLS, HB, APRIV, NV)                          \
    extern "C" __global__ __launch_bounds__(64 * WM * WN) void jv_gemm_##NAME##_##ROWS##x##COLS##r_g(GemmParams p) { \
        gemm_body<D, TM, TN, WM, WN, HB, APRIV, NV, true>(p);                                 \
    }
JV_GEMMG(q4k, DQ4K, 2, 4, 2, 2, 32, 64, true, true, 2)
JV_GEMMG(q6k, DF<FQ6K>, 2, 4, 2, 2, 32, 64, true, true, 2)
JV_GEMMG(q8_0, DF<FQ8_0Mix>, 2, 4, 2, 2, 32, 64, true, true, 2)
JV_GEMMG(q4k, DQ4K, 2, 8, 2, 2, 32, 128, true, true, 2)
JV_GEMMG(q6k, DF<FQ6K>, 2, 8, 2, 2, 32, 128, true, true, 2)
JV_GEMMG(q8_0, DF<FQ8_0Mix>, 2, 8, 2, 2, 32, 128, true, true, 2)
JV_GEMMG(q4k, DQ4K, 8, 8, 4, 2, 128, 128, true, true, 1)
JV_GEMMG(q6k, DF<FQ6K>, 8, 8, 4, 2, 128, 128, true, true, 1)
JV_GEMMG(q8_0, DF<FQ8_0>, 8, 8, 4, 2, 128, 128, true, true, 3)
JV_GEMMG(q4k, DQ4K, 16, 8, 8, 1, 256, 128, true, false, 4)
JV_GEMMG(q6k, DF<FQ6K>, 16, 8, 8, 1, 256, 128, true, false, 5)
JV_GEMMG(q8_0, DF<FQ8_0>, 16, 8, 4, 2, 256, 128, true, true, 3)
extern "C" __global__ __launch_bounds__(512) void jv_gemm_q4k_64x64r8(GemmParams p) { gemm8_body<DQ4K>(p); }
extern "C" __global__ __launch_bounds__(512) void jv_gemm_q4k_64x64r8_g(GemmParams p) { gemm8_body<DQ4K, true>(p); }
extern "C" __global__ __launch_bounds__(512) void jv_gemm_q6k_64x64r8_g(GemmParams p) { gemm8_body<DF<FQ6KMix>, true>(p); }
extern "C" __global__ __launch_bounds__(512) void jv_gemm_q8_0_64x64r8_g(GemmParams p) { gemm8_body<DF<FQ8_0Mix>, true>(p); }
extern "C" __global__ __launch_bounds__(512) void jv_gemm_q6k_64x64r8(GemmParams p) { gemm8_body<DF<FQ6KMix>>(p); }
extern "C" __global__ __launch_bounds__(512) void jv_gemm_q8_0_64x64r8(GemmParams p) { gemm8_body<DF<FQ8_0Mix>>(p); }
JV_GEMM_TILES(q4k, DQ4K)
JV_GEMM_TILES(q6k, DF<FQ6K>)
JV_GEMM_TILES(q8_0, DF<FQ8_0>)
JV_GEMM_TILES(q5_0, DF<FQ5_0>)
JV_GEMM_TILES(f16, DF<FF16>)

// ---------------------------------------------------------------------------------------------
// Repack GGML blocks (device copy) into the device layouts above.
// ---------------------------------------------------------------------------------------------

// One work item per Q4_K block row: 144 raw bytes -> its pieces of the tile layout.
extern "C" __global__ __launch_bounds__(256) void jv_repack_q4k(RepackParams p, int32_t kblocks) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;  // row * kblocks + u
    if (b >= p.chunks) return;
    const int64_t row = b / kblocks;
    const int64_t u = b - row * kblocks;
    const int rr = (int)(row & 15);
    const uint8_t *src = p.raw + b * 144;
    uint8_t *tb = p.wq + ((row >> 4) * kblocks + u) * 2304;
    *(uint4 *)(tb + 2048 + rr * 16) = *(const uint4 *)src;
    const int order[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    for (int g = 0; g < 4; ++g) {
        uint8_t piece[32];
        for (int pr = 0; pr < 4; ++pr)
            for (int e = 0; e < 8; ++e) piece[8 * pr + e] = src[16 + 32 * pr + 8 * g + order[e]];
        uint8_t *d0 = tb + (16 * g + rr) * 16, *d1 = tb + 1024 + (16 * g + rr) * 16;
        for (int e = 0; e < 16; ++e) {
            d0[e] = piece[e];
            d1[e] = piece[16 + e];
        }
    }
}

// One work item per Q6_K block row: 210 raw bytes -> its pieces of the tile layout.
extern "C" __global__ __launch_bounds__(256) void jv_repack_q6k(RepackParams p, int32_t kblocks) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;  // row * kblocks + u
    if (b >= p.chunks) return;
    const int64_t row = b / kblocks;
    const int64_t u = b - row * kblocks;
    const int rr = (int)(row & 15);
    const uint8_t *src = p.raw + b * 210;
    uint8_t *tb = p.wq + ((row >> 4) * kblocks + u) * 3360;
    const int order[4] = {0, 2, 1, 3};
    for (int g = 0; g < 4; ++g) {
        uint8_t o[48];
        for (int hf = 0; hf < 2; ++hf)
            for (int i2 = 0; i2 < 2; ++i2)
                for (int e = 0; e < 8; ++e) o[8 * (2 * hf + i2) + e] = src[64 * hf + 32 * i2 + 8 * g + e];
        for (int hf = 0; hf < 2; ++hf)
            for (int e = 0; e < 8; ++e) o[32 + 8 * hf + e] = src[128 + 32 * hf + 8 * g + e];
        for (int piece = 0; piece < 3; ++piece)
            for (int e = 0; e < 16; ++e)
                tb[1024 * piece + (16 * g + rr) * 16 + e] = o[16 * piece + (e & ~3) + order[e & 3]];
    }
    for (int e = 0; e < 16; ++e) tb[3072 + 16 * rr + e] = src[192 + e];
    tb[3328 + 2 * rr] = src[208];
    tb[3328 + 2 * rr + 1] = src[209];
}
// One work item per 64 k of a row (two Q8_0 blocks): 68 raw bytes -> its pieces of the tile layout.
extern "C" __global__ __launch_bounds__(256) void jv_repack_q8_0(RepackParams p, int32_t kchunks) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;  // row * kchunks + u
    if (c >= p.chunks) return;
    const int64_t row = c / kchunks;
    const int64_t u = c - row * kchunks;
    const int rr = (int)(row & 15);
    const uint8_t *src = p.raw + c * 68;
    uint8_t *tb = p.wq + ((row >> 4) * kchunks + u) * 1088;
    const int order[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    for (int g = 0; g < 4; ++g)
        for (int blk = 0; blk < 2; ++blk)
            for (int e = 0; e < 8; ++e)
                tb[(16 * g + rr) * 16 + 8 * blk + e] = (uint8_t)(src[34 * blk + 2 + 8 * g + order[e]] ^ 0x80u);
    for (int blk = 0; blk < 2; ++blk) {
        tb[1024 + 4 * rr + 2 * blk] = src[34 * blk];
        tb[1024 + 4 * rr + 2 * blk + 1] = src[34 * blk + 1];
    }
}
extern "C" __global__ __launch_bounds__(256) void jv_repack_q5_0(RepackParams p) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= p.chunks) return;
    const uint8_t *src = p.raw + c * 44;
    uint8_t *dst = p.wq + c * 32;
    for (int hb = 0; hb < 2; ++hb)
        for (int blk = 0; blk < 2; ++blk)
            for (int e = 0; e < 8; ++e) dst[16 * hb + 8 * blk + e] = src[22 * blk + 6 + 8 * hb + e];
    for (int blk = 0; blk < 2; ++blk) {
        for (int e = 0; e < 4; ++e) p.wh[8 * c + 4 * blk + e] = src[22 * blk + 2 + e];
        p.wd[4 * c + 2 * blk] = src[22 * blk];
        p.wd[4 * c + 2 * blk + 1] = src[22 * blk + 1];
    }
}

// ---------------------------------------------------------------------------------------------
// Row argmax with greedy's rule (crates/jevons-core/src/model.rs:207-219): the first maximum
// wins; any non-finite value makes the row invalid (-1).
// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
// lm_head consumers (crates/jevons-gemma4-diffusion/src/gpu/ops.rs:589-634, :750-758).
// ---------------------------------------------------------------------------------------------

// In-place final-logit soft capping: x = cap tanh(x / cap). Thread t handles x[4t .. 4t + 3]:
// one 16-byte load and store where x is 16-byte aligned, element by element otherwise and at
// the end of the buffer.
extern "C" __global__ __launch_bounds__(256) void jv_softcap(float *x, int64_t len, float cap) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= len) return;
    if (i + 4 <= len && ((uintptr_t)x & 15u) == 0) {
        float4 v = *(const float4 *)(x + i);
        v.x = soft_capped(v.x, cap);
        v.y = soft_capped(v.y, cap);
        v.z = soft_capped(v.z, cap);
        v.w = soft_capped(v.w, cap);
        *(float4 *)(x + i) = v;
    } else {
        for (int64_t j = i; j < len && j < i + 4; ++j) x[j] = soft_capped(x[j], cap);
    }
}

// One workgroup per (row, token) pair: thread i covers K unit i / 4 and lane group i % 4 of the
// table row, decoding its weights exactly in FP32 (the F decoders), then the workgroup sums the
// 256 partials in a fixed tree. A pair outside the activation rows or the table gives NaN.
template <class F>
__device__ __forceinline__ void pick_body(const PickParams &p) {
    __shared__ float part[256];
    const int pi = blockIdx.x;
    const uint32_t row = p.pairs[2 * pi], token = p.pairs[2 * pi + 1];
    const bool ok = row < (uint32_t)p.x_rows && token < (uint32_t)p.n;
    float acc = 0.f;
    if (ok) {
        const int U = p.d / F::KU;
        for (int i = threadIdx.x; i < U * 4; i += 256) {
            const int u = i >> 2, g = i & 3;
            typename F::Raw raw;
            typename F::Prep pp;
            F::load(raw, p.wq, p.wh, p.wd, p.d, (int)token, u, g);
            F::prep(raw, pp, g);
#pragma unroll
            for (int s = 0; s < F::KU / 32; ++s) {
                float v[8];
                F::frag_f32(raw, pp, s, g, v);
                const size_t c = (size_t)row * (size_t)p.d + (size_t)(u * F::KU + F::kidx(s, g));
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float xv = p.act == 0 ? h2f(((const uint16_t *)p.x)[c + e])
                                   : p.act == 1 ? bf2f(((const uint16_t *)p.x)[c + e])
                                                : ((const float *)p.x)[c + e];
                    acc = __builtin_fmaf(v[e], xv, acc);
                }
            }
        }
    }
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) p.out[pi] = ok ? p.cap * tanhf(part[0] / p.cap) : __builtin_nanf("");
}

#define JV_PICK(NAME, F) \
    extern "C" __global__ __launch_bounds__(256) void jv_pick_logits_##NAME(PickParams p) { pick_body<F>(p); }
JV_PICK(q4k, FQ4K)
JV_PICK(q6k, FQ6K)
JV_PICK(q8_0, FQ8_0)
JV_PICK(q5_0, FQ5_0)
JV_PICK(f16, FF16)

// Expert grouping (ops::group, crates/jevons-gemma4-diffusion/src/gpu/ops.rs:522-587), one
// workgroup: sorted[] lists the assignments of expert 0, then 1, ... (each in assignment order),
// offsets[e] is expert e's first sorted position (offsets[experts] = routed count), jobs[0] the
// number of bm-row tiles and jobs[1 + 2j], jobs[2 + 2j] tile j's (expert, first position).
// Ids >= experts are not routed; experts <= 1024.
extern "C" __global__ __launch_bounds__(1024) void jv_group_routes(const uint32_t *ids, uint32_t assignments,
                                                                  uint32_t experts, uint32_t bm,
                                                                  uint32_t *sorted, uint32_t *offsets,
                                                                  uint32_t *jobs) {
    // A stable counting sort in one workgroup of NW waves. Wave w owns the contiguous
    // assignments [a0, a1): it counts them per expert, the counts become per-wave starting
    // positions (expert start + the counts of earlier waves), and the wave places its
    // assignments in order, ranking the lanes of one expert within each 64-assignment batch.
    // So every expert's positions hold its assignments in increasing order. The lanes holding
    // the same expert come from one ballot per bit of the expert id (same_expert), so a batch
    // costs a fixed handful of instructions however many experts it touches.
    constexpr int NW = 16;
    __shared__ uint32_t cnt[NW][1024];
    __shared__ uint32_t starts[1025], jst[1025];
    const int tid = (int)threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid; i < NW * 1024; i += 64 * NW) cnt[i >> 10][i & 1023] = 0;
    __syncthreads();
    const uint32_t per = (assignments + NW - 1) / NW;
    const uint32_t a0 = min((uint32_t)wv * per, assignments), a1 = min(a0 + per, assignments);
    // the lanes of this wave whose routed expert equals the lane's own (ex < experts)
    auto same_expert = [&](uint32_t ex, bool todo) {
        uint64_t same = __ballot(todo);
        for (uint32_t b = 0; (1u << b) < experts; ++b) {  // wave-uniform
            const bool bit = ((ex >> b) & 1u) != 0;
            const uint64_t ones = __ballot(todo && bit);
            same &= bit ? ones : ~ones;
        }
        return same;
    };
    for (uint32_t c = a0; c < a1; c += 64) {
        const uint32_t a = c + (uint32_t)lane;
        const uint32_t ex = a < a1 ? ids[a] : 0xffffffffu;
        const bool todo = ex < experts;
        const uint64_t same = same_expert(ex, todo);
        // the lowest lane of each expert adds the expert's count (one writer per entry)
        if (todo && (same & ((1ull << lane) - 1)) == 0) cnt[wv][ex] += (uint32_t)__popcll(same);
    }
    __syncthreads();
    for (uint32_t ex = (uint32_t)tid; ex < experts; ex += 64 * NW) {  // counts -> wave prefixes
        uint32_t sum = 0;
        for (int w = 0; w < NW; ++w) {
            const uint32_t c = cnt[w][ex];
            cnt[w][ex] = sum;
            sum += c;
        }
        starts[ex] = sum;
    }
    __syncthreads();
    if (wv == 0) {  // exclusive scans of the counts and job counts: lane l owns experts 16l..16l+15
        uint32_t c[16], jc[16], sum = 0, jsum = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t ex = 16u * (uint32_t)lane + (uint32_t)i;
            c[i] = ex < experts ? starts[ex] : 0u;
            jc[i] = (c[i] + bm - 1) / bm;
            sum += c[i];
            jsum += jc[i];
        }
        uint32_t incl = sum, jincl = jsum;  // inclusive prefix over lanes
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, d), jo = (uint32_t)__shfl_up((int)jincl, d);
            if (lane >= d) {
                incl += o;
                jincl += jo;
            }
        }
        uint32_t acc = incl - sum, jacc = jincl - jsum;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t ex = 16u * (uint32_t)lane + (uint32_t)i;
            if (ex < experts) {
                starts[ex] = acc;
                jst[ex] = jacc;
            }
            acc += c[i];
            jacc += jc[i];
        }
        if (lane == 63) {
            starts[experts] = incl;
            offsets[experts] = incl;
            jobs[0] = jincl;
        }
    }
    __syncthreads();
    for (uint32_t ex = (uint32_t)tid; ex < experts; ex += 64 * NW) {
        offsets[ex] = starts[ex];
        const uint32_t tiles = (starts[ex + 1] - starts[ex] + bm - 1) / bm;
        for (uint32_t t = 0; t < tiles; ++t) {
            jobs[1 + 2 * (jst[ex] + t)] = ex;
            jobs[2 + 2 * (jst[ex] + t)] = starts[ex] + t * bm;
        }
    }
    for (uint32_t c = a0; c < a1; c += 64) {
        const uint32_t a = c + (uint32_t)lane;
        const uint32_t ex = a < a1 ? ids[a] : 0xffffffffu;
        const bool todo = ex < experts;
        const uint64_t same = same_expert(ex, todo);
        const uint32_t rank = (uint32_t)__popcll(same & ((1ull << lane) - 1));
        uint32_t base = 0;
        if (todo) base = starts[ex] + cnt[wv][ex];  // every lane reads before any lane writes
        if (todo) {
            sorted[base + rank] = a;
            if (rank == 0) cnt[wv][ex] = base - starts[ex] + (uint32_t)__popcll(same);
        }
    }
}

// (max, index) of a wave's lanes under better(); every lane ends with the result.
__device__ __forceinline__ void wave_best(float &v, int &i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi = __shfl_xor(i, off);
        better(v, i, ov, oi);
    }
}

// (max, index) of a workgroup of up to 16 waves; thread 0 holds the result. `bad` is or-ed the
// same way.
__device__ __forceinline__ void group_best(float &v, int &i, int &bad) {
    __shared__ float sv[16];
    __shared__ int si[16], sb[16];
    wave_best(v, i);
    bad = __any(bad) ? 1 : 0;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = v;
        si[wave] = i;
        sb[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
            better(v, i, sv[w], si[w]);
            bad |= sb[w];
        }
    }
}

// Grid (chunks, rows), 256 threads: partial (max, index) of logits[row][c chunk, min(n, (c + 1)
// chunk)), index -1 when that range holds a non-finite value (greedy's error,
// crates/jevons-core/src/model.rs:207-219). `vec` (rows 16-byte aligned, chunk a multiple of
// 1024): each thread loads chunk / 1024 float4 at once; otherwise scalar loads.
extern "C" __global__ __launch_bounds__(256) void jv_argmax_partial(const float *logits, int64_t n,
                                                                   int chunk, int vec, float *pval,
                                                                   int *pidx) {
    const int row = blockIdx.y;
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    const int64_t c1 = min(c0 + (int64_t)chunk, n);
    const float *src = logits + (int64_t)row * n;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    int bad = 0;
    if (vec) {
        constexpr int kMaxLoads = 4;  // chunk <= 4096
        const int loads = chunk >> 10;
        float4 v[kMaxLoads];
#pragma unroll
        for (int j = 0; j < kMaxLoads; ++j) {
            const int64_t e = c0 + 4 * ((int64_t)j * 256 + threadIdx.x);
            if (j < loads && e < c1) v[j] = *(const float4 *)(src + e);
        }
#pragma unroll
        for (int j = 0; j < kMaxLoads; ++j) {
            const int64_t e = c0 + 4 * ((int64_t)j * 256 + threadIdx.x);
            if (j < loads && e < c1) {
                const float x[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bad |= !__builtin_isfinite(x[q]);
                    better(bv, bi, x[q], (int)(e + q));
                }
            }
        }
    } else {
        for (int64_t e = c0 + threadIdx.x; e < c1; e += 256) {
            const float x = src[e];
            bad |= !__builtin_isfinite(x);
            better(bv, bi, x, (int)e);
        }
    }
    group_best(bv, bi, bad);
    if (threadIdx.x == 0) {
        const int64_t o = (int64_t)row * gridDim.x + blockIdx.x;
        pval[o] = bv;
        pidx[o] = bad ? -1 : bi;
    }
}

// Grid (rows), 256 to 1024 threads (a multiple of 64): combine the partials of each row; -1 if
// any range was non-finite or the row is empty. Each thread issues the loads of eight partials
// before it compares them (a row's thousands of partials in one round trip). Partials past the
// row's end read as (-inf, INT_MAX), which never replaces a result: valid partials are finite.
extern "C" __global__ __launch_bounds__(1024) void jv_argmax_final(const float *pval, const int *pidx,
                                                                   int chunks, int *index) {
    const int row = blockIdx.x;
    const float *pv = pval + (int64_t)row * chunks;
    const int *pi = pidx + (int64_t)row * chunks;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    int bad = 0;
    constexpr int kBatch = 8;
    const int nt = (int)blockDim.x;
    for (int c0 = 0; c0 < chunks; c0 += nt * kBatch) {
        float v[kBatch];
        int i[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int c = c0 + j * nt + (int)threadIdx.x;
            const bool in = c < chunks;
            v[j] = in ? pv[c] : -__builtin_inff();
            i[j] = in ? pi[c] : 0x7fffffff;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            if (i[j] < 0)
                bad = 1;
            else
                better(bv, bi, v[j], i[j]);
        }
    }
    group_best(bv, bi, bad);
    if (threadIdx.x == 0) index[row] = (bad || chunks == 0) ? -1 : bi;
}

// ---------------------------------------------------------------------------------------------
// Memory floor probe (benchmark only, not a product kernel): workgroup b reads the 16-byte units
// [b per, (b + 1) per) of src, each thread its units t, t + 512, ... with eight loads in flight,
// and folds them into one word. The word is stored only if it equals a value that the
// benchmark's inputs do not produce, so the loads cannot be dropped; sink holds one word per
// workgroup. Its duration is the time one launch takes to stream the same bytes as a product.
// ---------------------------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(512) void jv_probe_stream_read(const uint4 *src, int64_t units,
                                                                       int32_t per, uint32_t *sink) {
    const int64_t base = (int64_t)blockIdx.x * per;
    const int64_t end = min(base + (int64_t)per, units);
    uint32_t acc = 0;
    constexpr int kInFlight = 8;
    for (int64_t i0 = base + threadIdx.x; i0 < end; i0 += kInFlight * 512) {
        uint4 v[kInFlight];
#pragma unroll
        for (int j = 0; j < kInFlight; ++j) {
            const int64_t i = i0 + (int64_t)j * 512;
            v[j] = i < end ? src[i] : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < kInFlight; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (acc == 0x8badf00du) sink[blockIdx.x] = acc;
}

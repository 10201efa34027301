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

#include "../qmm_params.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kLdsPad = 8;  // FP16 elements of padding per staged activation row (16 bytes)

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

__device__ __forceinline__ f16x8 pack8(const float v[8]) {
    f16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)v[e];
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

// Q4_K, device layout = the GGUF blocks unchanged: row-major [rows][K/256] x 144 bytes
// (f16 d, f16 dmin, 12 scale bytes, 128 quant bytes). Lane group g holds pair g of the block
// (quant bytes 32g..32g+31): step s = 4h + c covers bytes 8c..8c+7, nibble h, i.e. elements
// 64g + 32h + 8c + e of sub-block 2g + h (quant.rs:25-41).
struct FQ4K {
    static constexpr int KU = 256;
    struct Raw {
        uint4 hd, q0, q1;
    };
    struct Prep {
        float dd[2], mm[2];
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *,
                                int K, int row, int u, int g) {
        const uint8_t *blk = wq + ((size_t)row * (size_t)(K / 256) + (size_t)u) * 144u;
        r.hd = ld16(blk);
        r.q0 = ld16(blk + 16 + 32 * g);
        r.q1 = ld16(blk + 32 + 32 * g);
    }
    // q4k_scale_min (quant.rs:14-23) for sub-blocks j = 2g and 2g + 1.
    __device__ static void prep(const Raw &r, Prep &p, int g) {
        const float d = h2f(r.hd.x), dmin = h2f(r.hd.x >> 16);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * g + h;
            const int jj = j & 3;
            const uint32_t a = (r.hd.y >> (8 * jj)) & 0xffu;  // scale byte jj
            const uint32_t b = (r.hd.z >> (8 * jj)) & 0xffu;  // scale byte jj + 4
            const uint32_t c = (r.hd.w >> (8 * jj)) & 0xffu;  // scale byte jj + 8
            uint32_t sc, mn;
            if (j < 4) {
                sc = a & 63u;
                mn = b & 63u;
            } else {
                sc = (c & 15u) | ((a >> 6) << 4);
                mn = (c >> 4) | ((b >> 6) << 4);
            }
            p.dd[h] = d * (float)sc;     // exact: 11 x 6 significant bits
            p.mm[h] = dmin * (float)mn;  // exact
        }
    }
    __device__ static int kidx(int s, int g) { return 64 * g + 32 * (s >> 2) + 8 * (s & 3); }
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int, float v[8]) {
        const int h = s >> 2, c = s & 3;
        const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t ta = (w[2 * c] >> (4 * h)) & 0x0f0f0f0fu;
        const uint32_t tb = (w[2 * c + 1] >> (4 * h)) & 0x0f0f0f0fu;
        const float dd = p.dd[h], mm = p.mm[h];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // d*s*q is exact, so one fused rounding equals quant.rs's product-then-subtract.
            v[e] = __builtin_fmaf((float)((ta >> (8 * e)) & 0xffu), dd, -mm);
            v[e + 4] = __builtin_fmaf((float)((tb >> (8 * e)) & 0xffu), dd, -mm);
        }
    }
};

// Q6_K, device layout: per block 208 bytes + one FP16 scale in the d region.
// Bytes 48g..48g+47 hold lane group g's quants: ql(hf, i2) = ql[64hf + 32i2 + 8g, +8) for
// (hf, i2) = (0,0), (0,1), (1,0), (1,1), then qh(hf) = qh[32hf + 8g, +8) for hf = 0, 1;
// bytes 192..207 are the 16 int8 sub-block scales. Step s = 4hf + i covers elements
// 128hf + 32i + 8g + e (quant.rs:43-61).
struct FQ6K {
    static constexpr int KU = 256;
    struct Raw {
        uint4 a, b, c, sc;
        uint32_t d;
    };
    struct Prep {
        float d;
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *wd,
                                int K, int row, int u, int g) {
        const size_t blk_i = (size_t)row * (size_t)(K / 256) + (size_t)u;
        const uint8_t *blk = wq + blk_i * 208u;
        r.a = ld16(blk + 48 * g);
        r.b = ld16(blk + 48 * g + 16);
        r.c = ld16(blk + 48 * g + 32);
        r.sc = ld16(blk + 192);
        r.d = *(const uint16_t *)(wd + blk_i * 2u);
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
        for (int e = 0; e < 8; ++e) {
            const uint32_t ql = w[qi + (e >> 2)] >> (8 * (e & 3) + nib);
            const uint32_t qh = w[hi + (e >> 2)] >> (8 * (e & 3) + 2 * i);
            const int32_t q = (int32_t)((ql & 15u) | ((qh & 3u) << 4)) - 32;
            v[e] = scale * (float)q;  // (d * sc) * q, as quant.rs evaluates it
        }
    }
};

// Q8_0, device layout: per 64 k (two blocks) 64 quant bytes; bytes 16g..16g+15 hold
// block0[8g, +8) then block1[8g, +8). FP16 scales per block in the d region.
// Step s (0, 1) is block s; elements 32s + 8g + e (quant.rs:75-80).
struct FQ8_0 {
    static constexpr int KU = 64;
    struct Raw {
        uint4 q;
        uint32_t d2;
    };
    struct Prep {
        float d[2];
    };
    __device__ static void load(Raw &r, const uint8_t *wq, const uint8_t *, const uint8_t *wd,
                                int K, int row, int u, int g) {
        const size_t ch = (size_t)row * (size_t)(K / 64) + (size_t)u;
        r.q = ld16(wq + ch * 64u + 16 * g);
        r.d2 = *(const uint32_t *)(wd + ch * 4u);
    }
    __device__ static void prep(const Raw &r, Prep &p, int) {
        p.d[0] = h2f(r.d2);
        p.d[1] = h2f(r.d2 >> 16);
    }
    __device__ static int kidx(int s, int g) { return 32 * s + 8 * g; }
    __device__ static void frag_f32(const Raw &r, const Prep &p, int s, int, float v[8]) {
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int32_t q = (int32_t)(int8_t)((w[2 * s + (e >> 2)] >> (8 * (e & 3))) & 0xffu);
            v[e] = p.d[s] * (float)q;
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
// Activation staging: rows [m0, m0 + rows) x k [k0, k0 + kl) -> LDS FP16, row stride `stride`.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void stage_rows(const QmmParams &p, _Float16 *lds, int m0, int rows,
                                           int k0, int kl, int stride) {
    const int per_row = kl >> 3;
    const int total = rows * per_row;
    for (int i = threadIdx.x; i < total; i += kThreads) {
        const int r = i / per_row;
        const int c8 = i - r * per_row;
        const size_t src = (size_t)(m0 + r) * (size_t)p.ldx + (size_t)(k0 + 8 * c8);
        f16x8 v;
        if (p.act == 0) {
            v = __builtin_bit_cast(f16x8, *(const uint4 *)((const uint16_t *)p.x + src));
        } else if (p.act == 1) {
            const uint4 b = *(const uint4 *)((const uint16_t *)p.x + src);
            const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = (_Float16)bf2f(w[e]);
                v[2 * e + 1] = (_Float16)bf2f(w[e] >> 16);
            }
        } else {
            const float4 a = *(const float4 *)((const float *)p.x + src);
            const float4 b = *(const float4 *)((const float *)p.x + src + 4);
            v[0] = (_Float16)a.x; v[1] = (_Float16)a.y; v[2] = (_Float16)a.z; v[3] = (_Float16)a.w;
            v[4] = (_Float16)b.x; v[5] = (_Float16)b.y; v[6] = (_Float16)b.z; v[7] = (_Float16)b.w;
        }
        *(f16x8 *)(lds + r * stride + 8 * c8) = v;
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
    const int m0 = (int)blockIdx.y * 16 * MT;
    const bool active = n_base < p.N;
    const int rows_real = min(16 * MT, p.M - m0);
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
            F::load(cur[t], p.wq, p.wh, p.wd, p.K, n_base + 16 * t + r16, u_first, g);
    }

    int chunk_u0 = u_first;
    for (int u = u_first; u < u_last; ++u) {
        if ((u - u_first) % kc_units == 0) {
            chunk_u0 = u;
            const int kl = min(kc_units, u_last - u) * F::KU;
            __syncthreads();
            stage_rows(p, lds, m0, rows_real, u * F::KU, kl, stride);
            __syncthreads();
        }
        if (active) {
            if (u + 1 < u_last) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    F::load(nxt[t], p.wq, p.wh, p.wd, p.K, n_base + 16 * t + r16, u + 1, g);
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
            const int row = m0 + mt * 16 + 4 * g + i;
            if (row >= p.M) continue;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int col = n_base + 16 * t + r16;
                const float v = acc[mt][t][i];
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

}  // namespace

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

// ---------------------------------------------------------------------------------------------
// Repack GGML blocks (device copy) into the device layouts above.
// ---------------------------------------------------------------------------------------------

// One work item per Q6_K block: 210 raw bytes -> 208 layout bytes + FP16 scale.
extern "C" __global__ __launch_bounds__(256) void jv_repack_q6k(RepackParams p) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= p.chunks) return;
    const uint8_t *src = p.raw + b * 210;
    uint8_t *dst = p.wq + b * 208;
    for (int g = 0; g < 4; ++g) {
        uint8_t *o = dst + 48 * g;
        for (int hf = 0; hf < 2; ++hf)
            for (int i2 = 0; i2 < 2; ++i2)
                for (int e = 0; e < 8; ++e) o[8 * (2 * hf + i2) + e] = src[64 * hf + 32 * i2 + 8 * g + e];
        for (int hf = 0; hf < 2; ++hf)
            for (int e = 0; e < 8; ++e) o[32 + 8 * hf + e] = src[128 + 32 * hf + 8 * g + e];
    }
    for (int e = 0; e < 16; ++e) dst[192 + e] = src[192 + e];
    p.wd[2 * b] = src[208];
    p.wd[2 * b + 1] = src[209];
}

// One work item per pair of Q8_0 blocks (64 k of one row).
extern "C" __global__ __launch_bounds__(256) void jv_repack_q8_0(RepackParams p) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= p.chunks) return;
    const uint8_t *src = p.raw + c * 68;
    uint8_t *dst = p.wq + c * 64;
    for (int g = 0; g < 4; ++g)
        for (int blk = 0; blk < 2; ++blk)
            for (int e = 0; e < 8; ++e) dst[16 * g + 8 * blk + e] = src[34 * blk + 2 + 8 * g + e];
    for (int blk = 0; blk < 2; ++blk) {
        p.wd[4 * c + 2 * blk] = src[34 * blk];
        p.wd[4 * c + 2 * blk + 1] = src[34 * blk + 1];
    }
}

// One work item per pair of Q5_0 blocks (64 k of one row).
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
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    // (v, i) replaces (bv, bi) if larger, or equal with a lower index.
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Grid (chunks, rows): partial (max, index) of logits[row][c*chunk, min(n, (c+1)*chunk)).
extern "C" __global__ __launch_bounds__(256) void jv_argmax_partial(const float *logits, int64_t n,
                                                                    int chunk, float *pval,
                                                                    int *pidx) {
    __shared__ float sv[256];
    __shared__ int si[256];
    __shared__ int sbad[256];
    const int row = blockIdx.y;
    const int c = blockIdx.x;
    const int64_t lo = (int64_t)c * chunk;
    const int64_t hi = min(n, lo + chunk);
    const float *x = logits + (int64_t)row * n;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    int bad = 0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
        const float v = x[i];
        if (!__builtin_isfinite(v)) bad = 1;
        better(bv, bi, v, (int)i);
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    sbad[threadIdx.x] = bad;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) {
            better(sv[threadIdx.x], si[threadIdx.x], sv[threadIdx.x + w], si[threadIdx.x + w]);
            sbad[threadIdx.x] |= sbad[threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int64_t o = (int64_t)row * gridDim.x + c;
        pval[o] = sv[0];
        pidx[o] = sbad[0] ? -1 : si[0];
    }
}

// Grid (rows): combine the partials of each row.
extern "C" __global__ __launch_bounds__(256) void jv_argmax_final(const float *pval, const int *pidx,
                                                                  int chunks, int *index) {
    __shared__ float sv[256];
    __shared__ int si[256];
    __shared__ int sbad[256];
    const int row = blockIdx.x;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    int bad = 0;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        const int i = pidx[(int64_t)row * chunks + c];
        if (i < 0)
            bad = 1;
        else
            better(bv, bi, pval[(int64_t)row * chunks + c], i);
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    sbad[threadIdx.x] = bad;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) {
            better(sv[threadIdx.x], si[threadIdx.x], sv[threadIdx.x + w], si[threadIdx.x + w]);
            sbad[threadIdx.x] |= sbad[threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) index[row] = (sbad[0] || chunks == 0) ? -1 : si[0];
}

// Host side of the gfx950 quantized GGML products: device client, weight upload and layout,
// launch plans, and the C ABI declared in include/jevons_qmm.h.
//
// This is the C++ counterpart of crates/jevons-kernels/src/{lib.rs,gemm.rs}: it validates every
// shape and buffer length on the host (the reference relies on CubeCL's checked launches and
// launch asserts), loads the kernels from a gfx950 code object with hipModule*, and launches
// them on the caller's stream.

#include "jevons_qmm.h"

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../qmm_params.h"

// Fixed device array of jv_matmul_noalloc (noalloc.hip): set-up on the current device, and the
// address kept for a device.
extern "C" hipError_t jv_internal_noalloc_setup(int device, size_t zero_bytes, void **out);
extern "C" void *jv_internal_noalloc_ptr(int device, hipError_t *status);

namespace {

thread_local std::string g_error;

jv_status fail(jv_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return st;
}

#define JV_HIP(call)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            return fail(e_ == hipErrorOutOfMemory ? JV_ERR_NO_MEMORY : JV_ERR_HIP, "%s: %s", \
                        #call, hipGetErrorString(e_));                                       \
    } while (0)

// GGML type table (crates/jevons-formats/src/gguf.rs:120-144).
bool type_block(uint32_t id, uint32_t *elems, uint32_t *bytes) {
    switch (id) {
    case JV_GGML_F32: *elems = 1; *bytes = 4; return true;
    case JV_GGML_F16: *elems = 1; *bytes = 2; return true;
    case JV_GGML_Q5_0: *elems = 32; *bytes = 22; return true;
    case JV_GGML_Q8_0: *elems = 32; *bytes = 34; return true;
    case JV_GGML_Q4K: *elems = 256; *bytes = 144; return true;
    case JV_GGML_Q6K: *elems = 256; *bytes = 210; return true;
    default: return false;
    }
}

// The reference's `{kind:?}` spelling of a type id.
std::string type_name(uint32_t id) {
    switch (id) {
    case JV_GGML_F32: return "F32";
    case JV_GGML_F16: return "F16";
    case JV_GGML_Q5_0: return "Q5_0";
    case JV_GGML_Q8_0: return "Q8_0";
    case JV_GGML_Q4K: return "Q4K";
    case JV_GGML_Q6K: return "Q6K";
    default: return "Other(" + std::to_string(id) + ")";
    }
}

const char *fmt_kernel_name(jv_fmt f) {
    switch (f) {
    case JV_FMT_Q4K: return "q4k";
    case JV_FMT_Q6K: return "q6k";
    case JV_FMT_Q5_0: return "q5_0";
    case JV_FMT_Q8_0: return "q8_0";
    default: return "f16";
    }
}

// K elements per kernel unit of a format (the decoders' KU).
int fmt_unit(jv_fmt f) { return (f == JV_FMT_Q4K || f == JV_FMT_Q6K) ? 256 : 64; }

std::string library_dir() {
    Dl_info info;
    if (dladdr((void *)&jv_open, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t s = p.rfind('/');
        if (s != std::string::npos) return p.substr(0, s);
    }
    return ".";
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// IEEE binary16 <-> binary32 on the host (round to nearest even), for packed-scale checks.
uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    const int32_t e = (int32_t)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t full = man | 0x800000u, shift = (uint32_t)(14 - e);
        uint32_t q = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float f16_bits_to_f32(uint16_t b) {
    const uint32_t sign = (uint32_t)(b & 0x8000u) << 16, exp = (b >> 10) & 0x1fu, man = b & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        float v = (float)man * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 31) x = sign | 0x7f800000u | (man << 13);
    else x = sign | ((exp + 112u) << 23) | (man << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

}  // namespace

struct jv_ctx {
    int device = 0;
    hipModule_t module = nullptr;
    std::unordered_map<std::string, hipFunction_t> fns;
    jv_device_info info{};
    void *pack = nullptr;  // packed activation fragments of the pipelined tiles (grows)
    size_t pack_bytes = 0;
    jv_scratch *own = nullptr;  // split-K small-row scratch of products given none (grows)
    // greedy epilogue state of jv_matmul_argmax (grows, zeroed when allocated; each call
    // leaves what it used at zero): per row a flag and a key
    void *greedy = nullptr;
    size_t greedy_rows = 0;
    // Buffers replaced by a larger one. A HIP graph captured before the growth still holds their
    // addresses, so they stay allocated until the context is closed.
    std::vector<void *> retired;
};

struct jv_qmatrix {
    jv_ctx *ctx = nullptr;
    uint32_t ggml_type = 0;
    jv_fmt fmt = JV_FMT_Q4K;
    size_t n = 0, k = 0, experts = 1;
    uint8_t *base = nullptr;  // owned allocation holding every region (null for views)
    const uint8_t *q = nullptr, *h = nullptr, *d = nullptr;
    size_t bytes = 0;
};

struct jv_scratch {
    jv_ctx *ctx = nullptr;
    void *buf = nullptr;
    size_t bytes = 0;
    std::vector<void *> retired;  // smaller buffers kept for graphs captured on them
    bool fixed = false;  // the fixed array of jv_matmul_noalloc: never grows, never freed here
};

namespace {

// Every scratch allocation starts with the split-K small-row kernels' tile counters (zeroed when
// allocated, a multiple of 16 after every launch); partial buffers of all uses follow them.
constexpr size_t kCounterTiles = 65536;
constexpr size_t kCounterBytes = kCounterTiles * 4;

// Size of a grown buffer: at least twice the old one, so that the buffers a context retires
// over its life add up to less than its largest one.
size_t grown_size(size_t old_bytes, size_t need) { return std::max(need, 2 * old_bytes); }

// Grows `s` to hold `payload` bytes after the counters and returns the payload's address. The
// replaced buffer is retired, not freed: launches captured in a HIP graph keep its address.
jv_status scratch_reserve(jv_scratch *s, size_t payload, void **out) {
    const size_t need = kCounterBytes + payload;
    if (s->fixed && s->bytes < need)
        return fail(JV_ERR_INVALID,
                    "the product needs %zu bytes of staging; the fixed scratch array holds %zu "
                    "(JV_NOALLOC_SCRATCH_BYTES, %zu of them tile counters)",
                    payload, s->bytes - kCounterBytes, kCounterBytes);
    if (s->bytes < need) {
        const size_t size = grown_size(s->bytes, need);
        void *buf = nullptr;
        JV_HIP(hipMalloc(&buf, size));
        hipError_t e = hipMemset(buf, 0, kCounterBytes);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            hipFree(buf);
            return fail(JV_ERR_HIP, "scratch counters: %s", hipGetErrorString(e));
        }
        if (s->buf) s->retired.push_back(s->buf);
        s->buf = buf;
        s->bytes = size;
    }
    *out = (uint8_t *)s->buf + kCounterBytes;
    return JV_OK;
}

jv_status get_fn(jv_ctx *ctx, const std::string &name, hipFunction_t *out) {
    auto it = ctx->fns.find(name);
    if (it != ctx->fns.end()) {
        *out = it->second;
        return JV_OK;
    }
    hipFunction_t f = nullptr;
    hipError_t e = hipModuleGetFunction(&f, ctx->module, name.c_str());
    if (e != hipSuccess)
        return fail(JV_ERR_NO_KERNELS, "kernel %s is missing from the code object: %s",
                    name.c_str(), hipGetErrorString(e));
    ctx->fns.emplace(name, f);
    *out = f;
    return JV_OK;
}

jv_status launch(jv_ctx *ctx, const std::string &name, dim3 grid, dim3 block, size_t lds,
                 void *stream, void **args) {
    hipFunction_t f;
    jv_status st = get_fn(ctx, name, &f);
    if (st != JV_OK) return st;
    JV_HIP(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                 (unsigned)lds, (hipStream_t)stream, args, nullptr));
    return JV_OK;
}

jv_status use_device(jv_ctx *ctx) {
    if (!ctx) return fail(JV_ERR_INVALID, "null context");
    JV_HIP(hipSetDevice(ctx->device));
    return JV_OK;
}

// Device bytes of each region of the gfx950 layout for `blocks` GGML blocks.
struct Layout {
    size_t q = 0, h = 0, d = 0;
};

Layout layout_for(jv_fmt fmt, size_t blocks) {
    Layout l;
    switch (fmt) {
    case JV_FMT_Q4K: l.q = blocks * 144; break;
    case JV_FMT_Q6K: l.q = blocks * 210; break;
    case JV_FMT_Q8_0: l.q = blocks * 34; break;
    case JV_FMT_Q5_0: l.q = blocks * 16; l.h = blocks * 4; l.d = blocks * 2; break;
    default: break;
    }
    return l;
}

// QMatrix::upload / from_packed shape rules (gemm.rs:822-886), up to the weight format.
jv_status check_upload(uint32_t type, size_t n, size_t k, size_t experts, size_t bytes,
                       jv_fmt *fmt_out) {
    uint32_t block, size;
    if (!type_block(type, &block, &size)) return fail(JV_ERR_UNSUPPORTED, "unsupported type");
    const std::string kind = type_name(type);
    if (bytes != experts * n * k / block * size)
        return fail(JV_ERR_INVALID, "%s [%zux%zu, %zu] has the wrong byte count", kind.c_str(),
                    experts, n, k);
    if (bytes % size != 0)
        return fail(JV_ERR_INVALID, "tensor is not a whole number of blocks");
    jv_fmt fmt;
    switch (type) {
    case JV_GGML_Q4K: fmt = JV_FMT_Q4K; break;
    case JV_GGML_Q6K: fmt = JV_FMT_Q6K; break;
    case JV_GGML_Q5_0: fmt = JV_FMT_Q5_0; break;
    case JV_GGML_Q8_0: fmt = JV_FMT_Q8_0; break;
    default: return fail(JV_ERR_UNSUPPORTED, "%s has no GPU block layout", kind.c_str());
    }
    if (k % 64 != 0 || n % 64 != 0 || k % block != 0)
        return fail(JV_ERR_INVALID, "%s [%zux%zu, %zu] has an unsupported shape", kind.c_str(),
                    experts, n, k);
    if (experts == 0 || n * experts > (size_t)INT32_MAX || k > (size_t)INT32_MAX / 64)
        return fail(JV_ERR_INVALID, "%s [%zux%zu, %zu] has an unsupported shape", kind.c_str(),
                    experts, n, k);
    *fmt_out = fmt;
    return JV_OK;
}

// Lays out raw GGML blocks already in device memory (raw_dev) into a new matrix.
jv_status build_from_device(jv_ctx *ctx, uint32_t type, jv_fmt fmt, size_t n, size_t k,
                            size_t experts, const void *raw_dev, size_t bytes, jv_qmatrix **out) {
    uint32_t block, size;
    type_block(type, &block, &size);
    const size_t blocks = bytes / size;
    Layout l = layout_for(fmt, blocks);
    const size_t oq = 0, oh = align_up(l.q, 256), od = oh + align_up(l.h, 256);
    const size_t total = std::max<size_t>(od + align_up(l.d, 256), 256);
    uint8_t *base = nullptr;
    JV_HIP(hipMalloc((void **)&base, total));
    auto *w = new jv_qmatrix();
    w->ctx = ctx;
    w->ggml_type = type;
    w->fmt = fmt;
    w->n = n;
    w->k = k;
    w->experts = experts;
    w->base = base;
    w->q = base + oq;
    w->h = base + oh;
    w->d = base + od;
    w->bytes = l.q + l.h + l.d;
    jv_status st = JV_OK;
    if (fmt == JV_FMT_Q4K) {
        RepackParams rp{};
        rp.raw = (const uint8_t *)raw_dev;
        rp.wq = base + oq;
        rp.chunks = (int64_t)blocks;
        int32_t kblocks = (int32_t)(k / 256);
        void *args[] = {&rp, &kblocks};
        st = launch(ctx, "jv_repack_q4k", dim3((unsigned)((rp.chunks + 255) / 256)), dim3(256), 0,
                    nullptr, args);
        if (st == JV_OK) {
            hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) st = fail(JV_ERR_HIP, "repack: %s", hipGetErrorString(e));
        }
    } else {
        RepackParams rp{};
        rp.raw = (const uint8_t *)raw_dev;
        rp.wq = base + oq;
        rp.wh = base + oh;
        rp.wd = base + od;
        const char *name = nullptr;
        int32_t kchunks = 0;
        void *args[2] = {&rp, nullptr};
        if (fmt == JV_FMT_Q6K) {
            rp.chunks = (int64_t)blocks;
            name = "jv_repack_q6k";
            kchunks = (int32_t)(k / 256);
            args[1] = &kchunks;
        } else if (fmt == JV_FMT_Q8_0) {
            rp.chunks = (int64_t)(blocks / 2);
            name = "jv_repack_q8_0";
            kchunks = (int32_t)(k / 64);
            args[1] = &kchunks;
        } else {
            rp.chunks = (int64_t)(blocks / 2);
            name = "jv_repack_q5_0";
        }
        dim3 grid((unsigned)((rp.chunks + 255) / 256));
        st = launch(ctx, name, grid, dim3(256), 0, nullptr, args);
        if (st == JV_OK) {
            hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) st = fail(JV_ERR_HIP, "repack: %s", hipGetErrorString(e));
        }
    }
    if (st != JV_OK) {
        hipFree(base);
        delete w;
        return st;
    }
    *out = w;
    return JV_OK;
}

void put_f16(std::vector<uint8_t> &raw, size_t at, float v) {
    uint16_t b = f32_to_f16_bits(v);
    raw[at] = (uint8_t)(b & 0xff);
    raw[at + 1] = (uint8_t)(b >> 8);
}

// Row tile of a plan -> kernel MT (16-row m-subtiles per workgroup).
int plan_mt(const jv_plan &p) { return p.bm == 0 ? 1 : (int)p.bm / 16; }
// Column tile -> NT (16-column n-subtiles per wave; 4 waves).
int plan_nt(const jv_plan &p) { return p.bm == 0 ? 1 : (int)p.bn / 64; }

bool act_ok(jv_act a) { return a == JV_ACT_F16 || a == JV_ACT_BF16 || a == JV_ACT_F32; }
bool out_ok(jv_out o) { return o == JV_OUT_F32 || o == JV_OUT_BF16; }

// Expert-grouped launch arguments (Groups, gemm.rs:955-966) plus the rows per job.
struct GroupArgs {
    const uint32_t *ids, *offsets, *jobs;
    size_t max_jobs;
    uint32_t in_div;
    uint32_t cap;
};

// The greedy epilogue asked of a product (jv_matmul_argmax): the soft cap, the indices' buffer
// and the context's greedy state; `done` tells whether the kernel the product took had the
// epilogue (and so wrote the indices).
struct GreedyArgs {
    float cap = 0.f;
    int32_t *index = nullptr;
    uint32_t *bad = nullptr;
    uint64_t *key = nullptr;
    bool done = false;
};

// jv_argmax_final over `rows` rows of `chunks` partials: one workgroup per row, of enough waves
// (4 to 16) that each thread loads at most eight partials at once where possible.
jv_status launch_argmax_final(jv_ctx *ctx, float *pval, int32_t *pidx, int chunks, size_t rows,
                              int32_t *index, void *stream) {
    const unsigned threads = (unsigned)std::min(1024, std::max(256, (chunks + 7) / 8 + 63) / 64 * 64);
    void *a2[] = {&pval, &pidx, &chunks, &index};
    return launch(ctx, "jv_argmax_final", dim3((unsigned)rows), dim3(threads), 0, stream, a2);
}

// The context's greedy state for at least `rows` rows, grown and zeroed as needed (a replaced
// buffer is retired): a flag per row, then from the next 256-byte boundary a key per row.
size_t greedy_keys_at(size_t rows) { return (rows * 4 + 255) & ~(size_t)255; }

jv_status greedy_state(jv_ctx *ctx, size_t rows, GreedyArgs *gr) {
    if (ctx->greedy_rows < rows) {
        const size_t cap = std::max(rows, 2 * ctx->greedy_rows);
        const size_t bytes = greedy_keys_at(cap) + cap * 8;
        void *buf = nullptr;
        JV_HIP(hipMalloc(&buf, bytes));
        hipError_t e = hipMemset(buf, 0, bytes);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            hipFree(buf);
            return fail(JV_ERR_HIP, "greedy state: %s", hipGetErrorString(e));
        }
        if (ctx->greedy) ctx->retired.push_back(ctx->greedy);
        ctx->greedy = buf;
        ctx->greedy_rows = cap;
    }
    uint8_t *base = (uint8_t *)ctx->greedy;
    gr->bad = (uint32_t *)base;
    gr->key = (uint64_t *)(base + greedy_keys_at(ctx->greedy_rows));
    return JV_OK;
}

// After a product with the greedy epilogue: jv_greedy_finish turns the folded keys of its `rows`
// rows into gr->index and zeroes them.
jv_status greedy_finish(jv_ctx *ctx, GreedyArgs *gr, size_t rows, void *stream) {
    int32_t *index = gr->index;
    int r = (int)rows;
    void *args[] = {&gr->key, &gr->bad, &index, &r};
    jv_status st = launch(ctx, "jv_greedy_finish", dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, args);
    if (st == JV_OK) gr->done = true;
    return st;
}

// Staging buffers of one product: `pack_bytes` of packed or converted activations (the context's
// buffer, grown as needed) and `part_bytes` of split-K partials (after the counters of
// `scratch`). With the fixed array of jv_matmul_noalloc both come from that array, one after
// the other, and nothing is allocated.
jv_status stage_buffers(jv_ctx *ctx, jv_scratch *scratch, size_t pack_bytes, size_t part_bytes,
                        void **pack, void **part) {
    *pack = nullptr;
    *part = nullptr;
    if (scratch && scratch->fixed) {
        const size_t at = align_up(pack_bytes, 256);
        void *payload = nullptr;
        jv_status st = scratch_reserve(scratch, at + part_bytes, &payload);
        if (st != JV_OK) return st;
        if (pack_bytes) *pack = payload;
        if (part_bytes) *part = (uint8_t *)payload + at;
        return JV_OK;
    }
    if (pack_bytes && ctx->pack_bytes < pack_bytes) {
        // the smaller buffer is retired, not freed (graphs captured on it keep its address)
        const size_t size = grown_size(ctx->pack_bytes, pack_bytes);
        void *buf = nullptr;
        JV_HIP(hipMalloc(&buf, size));
        if (ctx->pack) ctx->retired.push_back(ctx->pack);
        ctx->pack = buf;
        ctx->pack_bytes = size;
    }
    if (pack_bytes) *pack = ctx->pack;
    if (part_bytes) {
        if (!scratch) return fail(JV_ERR_INVALID, "split-K plans need a scratch buffer");
        return scratch_reserve(scratch, part_bytes, part);
    }
    return JV_OK;
}

// jv_pack_x: `rows` rows of x into FP16 MFMA fragments (mtiles 16-row tiles; grouped: per
// job, rows_cap rows each) or, with `rowmajor` (BF16 and FP32 only), into FP16 rows [rows][K];
// rscale receives every packed row's range factor.
jv_status launch_pack(jv_ctx *ctx, const void *x, jv_act act, size_t rows, size_t k, int mtiles,
                      int rowmajor, uint16_t *out, float *rscale, const GroupArgs *grp, uint32_t rows_cap,
                      void *stream) {
    PackXParams pk{};
    pk.x = x;
    pk.out = out;
    pk.rscale = rscale;
    pk.M = (int32_t)rows;
    pk.K = (int32_t)k;
    pk.ldx = (int32_t)k;
    pk.act = (int32_t)act;
    pk.mtiles = mtiles;
    pk.rowmajor = rowmajor;
    if (grp) {
        pk.ids = grp->ids;
        pk.offsets = grp->offsets;
        pk.jobs = grp->jobs;
        pk.grouped = 1;
        pk.in_div = (int32_t)grp->in_div;
        pk.rows_cap = (int32_t)rows_cap;
    }
    void *args[] = {&pk};
    if (act == JV_ACT_F16) {  // a copy thread per 128 values of a packed row
        const size_t waves = (size_t)mtiles * (k / 256) * 2;
        return launch(ctx, "jv_pack_x", dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, args);
    }
    // a workgroup per P rows, of the fewest waves (at most 16) that keep every thread at 8 chunks
    // or fewer: P = 1 for up to 512 rows of K <= 4096, 2 for up to 256 longer rows, else 4 (the
    // fastest of P = 1, 2, 4 per shape in kernel traces: M = 32 K = 3840 4.2 against 5.3 us,
    // M = 256 K = 15360 11.6 against 14.4 us, M = 4096 K = 3840 11.6 against 16.0 us; and on the
    // M = 512 K = 3840 GEMM with its product, interleaved, 77.4 against 78.5 us with P = 4)
    const size_t packed_rows = rowmajor ? rows : (size_t)mtiles * 16;
    const size_t P = k <= 4096 ? (packed_rows > 512 ? 4 : 1) : (packed_rows > 256 ? 4 : 2);
    const size_t chunks = k / 8;
    const size_t nw = std::min<size_t>(16, std::max<size_t>(4 / P, (chunks * P + 511) / 512));
    pk.rpw = (int32_t)P;
    return launch(ctx, "jv_pack_x", dim3((unsigned)((packed_rows + P - 1) / P)), dim3((unsigned)(64 * nw)), 0,
                  stream, args);
}

// The generic tile kernel (any plan, split-K through the scratch buffer and jv_reduce_splits).
// m = output rows; grouped launches cover grp->max_jobs jobs of at most grp->cap rows.
jv_status launch_tiles(jv_ctx *ctx, const void *x, jv_act act, size_t m, const jv_qmatrix *w,
                       void *out, jv_out out_type, jv_scratch *scratch, jv_plan plan, void *stream,
                       const GroupArgs *grp) {
    jv_status st = JV_OK;
    const int MT = plan_mt(plan), NT = plan_nt(plan);
    const int KU = fmt_unit(w->fmt);
    const int splits = (int)plan.splits;
    const int U = (int)(w->k / KU);
    const int max_units = (U + splits - 1) / splits;
    const int rows_alloc = (int)std::min<size_t>((size_t)(16 * MT), grp ? (size_t)grp->cap : m);
    // LDS budget for the staged activation chunk: whole K for small tiles when it fits.
    const size_t budget = MT == 1 ? 128 * 1024 : 80 * 1024;
    int kc_units = (int)((budget / (2 * (size_t)rows_alloc) - 8) / (size_t)KU);
    kc_units = std::max(1, std::min(kc_units, max_units));
    const int kc = kc_units * KU;
    const size_t lds = (size_t)rows_alloc * (size_t)(kc + 8) * 2;
    if (lds > ctx->info.lds_bytes)
        return fail(JV_ERR_INVALID, "tile needs %zu bytes of LDS, the device has %zu", lds,
                    ctx->info.lds_bytes);

    // BF16 and FP32 rows are converted once into FP16 rows divided by their range factors
    // (jv_pack_x, row-major): the kernel stages FP16 and multiplies each output row by
    // its input row's factor.
    const size_t in_rows = grp ? (m + grp->in_div - 1) / grp->in_div : m;
    const size_t conv_bytes = act == JV_ACT_F16 ? 0 : align_up(in_rows * w->k * 2, 256) + in_rows * 4;
    void *conv = nullptr, *partials = nullptr;
    st = stage_buffers(ctx, scratch, conv_bytes, splits > 1 ? (size_t)splits * m * w->n * 4 : 0, &conv,
                       &partials);
    if (st != JV_OK) return st;
    float *rscale = nullptr;
    if (conv) {
        rscale = (float *)((uint8_t *)conv + align_up(in_rows * w->k * 2, 256));
        st = launch_pack(ctx, x, act, in_rows, w->k, 0, 1, (uint16_t *)conv, rscale, nullptr, 0, stream);
        if (st != JV_OK) return st;
    }

    QmmParams p{};
    p.x = conv ? conv : x;
    p.wq = w->q;
    p.wh = w->h;
    p.wd = w->d;
    p.M = (int32_t)m;
    p.N = (int32_t)w->n;
    p.K = (int32_t)w->k;
    p.ldx = (int32_t)w->k;
    p.ldo = (int32_t)w->n;
    p.act = (int32_t)JV_ACT_F16;
    p.out_type = (int32_t)out_type;
    p.rscale = rscale;
    p.kc = kc;
    p.splits = splits;
    p.split_stride = (int64_t)(m * w->n);
    if (grp) {
        p.grouped = 1;
        p.ids = grp->ids;
        p.offsets = grp->offsets;
        p.jobs = grp->jobs;
        p.in_div = (int32_t)grp->in_div;
        p.rows_cap = (int32_t)grp->cap;
    }
    p.out = splits > 1 ? partials : out;
    char name[64];
    snprintf(name, sizeof name, "jv_qmm_%s_m%d_n%d", fmt_kernel_name(w->fmt), MT, NT);
    const size_t gy = grp ? grp->max_jobs : (m + 16 * MT - 1) / (16 * MT);
    dim3 grid((unsigned)(w->n / (size_t)(64 * NT)), (unsigned)gy, (unsigned)splits);
    void *args[] = {&p};
    st = launch(ctx, name, grid, dim3(256), lds, stream, args);
    if (st != JV_OK || splits == 1) return st;
    const void *part = p.out;
    int64_t len = (int64_t)(m * w->n);
    int sp = splits, ot = (int)out_type;
    void *rargs[] = {&part, &out, &len, &sp, &ot};
    return launch(ctx, "jv_reduce_splits", dim3((unsigned)((len + 255) / 256)), dim3(256), 0,
                  stream, rargs);
}

// Pipelined tile kernels (256 x 128, 128 x 128, 64 x 64, and 32 x 64 for Q4_K, Q6_K and Q8_0;
// whole K in 256-element blocks): activations -> packed FP16 fragments (per job when grouped),
// then the product. Every output element is the same MFMA chain as in the generic tile kernel,
// so the plans give the same bits.
bool reg_format(const jv_qmatrix *w) {
    return w->fmt == JV_FMT_Q4K || w->fmt == JV_FMT_Q6K || w->fmt == JV_FMT_Q8_0;
}

// The context's own scratch buffer, for products given none that need one.
jv_scratch *own_scratch(jv_ctx *ctx) {
    if (!ctx->own) {
        ctx->own = new jv_scratch();
        ctx->own->ctx = ctx;
    }
    return ctx->own;
}

// Split-K slices of the generic kernel (format units [z U / splits, (z + 1) U / splits)) that
// are whole 256-element blocks, so the pipelined tiles can run them with the same bits.
bool block_slices(const jv_qmatrix *w, uint32_t splits) {
    const size_t ku = (size_t)fmt_unit(w->fmt), units = w->k / ku;
    if (w->k % 256 != 0 || splits < 1 || w->k / 256 < splits) return false;
    for (size_t z = 1; z < splits; ++z)
        if (z * units / splits * ku % 256 != 0) return false;
    return true;
}

// Plans the pipelined tiles run (the others run the generic tiles): 256 x 128, 128 x 128 and
// 64 x 64 in every format, 32 x 64 and 32 x 128 for the register-tile formats.
bool pipelined_plan(const jv_qmatrix *w, jv_plan plan) {
    return w->k % 256 == 0 && block_slices(w, plan.splits) &&
           ((plan.bm == 256 && plan.bn == 128) || (plan.bm == 128 && plan.bn == 128) ||
            (plan.bm == 64 && plan.bn == 64) ||
            (reg_format(w) && plan.bm == 32 && (plan.bn == 64 || plan.bn == 128)));
}

// `scratch` holds the split-K partials (plans with splits > 1); when it is the fixed array of
// jv_matmul_noalloc, it also holds the packed activations in place of the context's buffer.
jv_status launch_pipelined(jv_ctx *ctx, const void *x, jv_act act, size_t m, const jv_qmatrix *w,
                           void *out, jv_out out_type, jv_plan plan, void *stream,
                           const GroupArgs *grp, jv_scratch *scratch = nullptr, GreedyArgs *gr = nullptr) {
    jv_status st = JV_OK;
    if (grp && plan.splits > 1) return fail(JV_ERR_INVALID, "grouped pipelined tiles do not split K");
    const int jobs_or_tiles = grp ? (int)grp->max_jobs : (int)((m + plan.bm - 1) / plan.bm);
    const int mtiles = jobs_or_tiles * (int)(plan.bm / 16);
    // the greedy epilogue exists on the register tiles of Q4_K, Q6_K and Q8_0 (ungrouped, whole
    // K, FP32 out; 64 x 64 on its 8-wave tile)
    const char *regenv = getenv("JV_GEMM_REG");
    const bool reg = reg_format(w) && (plan.bm == 32 || !(regenv && regenv[0] == '0'));
    const bool greedy = gr && !grp && plan.splits == 1 && reg && out_type == JV_OUT_F32;
    // fragments, then each packed row's range factor
    const size_t frag_bytes = (size_t)mtiles * 16 * w->k * 2;
    const size_t part_bytes = plan.splits > 1 ? (size_t)plan.splits * m * w->n * 4 : 0;
    void *pack = nullptr, *partials = nullptr;
    st = stage_buffers(ctx, scratch, frag_bytes + (size_t)mtiles * 16 * 4, part_bytes, &pack, &partials);
    if (st != JV_OK) return st;
    if (greedy) {
        st = greedy_state(ctx, m, gr);
        if (st != JV_OK) return st;
    }
    float *rscale = (float *)((uint8_t *)pack + frag_bytes);
    st = launch_pack(ctx, x, act, m, w->k, mtiles, 0, (uint16_t *)pack, rscale, grp, plan.bm, stream);
    if (st != JV_OK) return st;
    GemmParams gp{};
    gp.xa = (const uint16_t *)pack;
    gp.rscale = rscale;
    gp.wq = w->q;
    gp.wh = w->h;
    gp.wd = w->d;
    gp.out = out;
    gp.M = (int32_t)m;
    gp.N = (int32_t)(w->n);
    gp.K = (int32_t)w->k;
    gp.ldo = (int32_t)(w->n);
    gp.out_type = (int32_t)out_type;
    gp.splits = (int32_t)plan.splits;
    gp.part = (float *)partials;
    if (greedy) {
        gp.cap = gr->cap;
        gp.amax_key = gr->key;
        gp.amax_bad = gr->bad;
    }
    gp.split_stride = (int64_t)(m * w->n);
    if (grp) {
        gp.ids = grp->ids;
        gp.offsets = grp->offsets;
        gp.jobs = grp->jobs;
        gp.grouped = 1;
        gp.rows_cap = (int32_t)plan.bm;
    }
    void *gargs[] = {&gp};
    char name[40];
    // Q4_K, Q6_K and Q8_0 tiles run on waves that keep their activation fragments in
    // registers (same bits as the tiles that share them through LDS; JV_GEMM_REG=0 selects
    // those, except for 32 x 64, which exists only with register fragments): `reg` above.
    // Ungrouped 64 x 64 products run the 8-wave tile (two waves per SIMD) up to two workgroups
    // per CU; larger grids and expert jobs the 4-wave one, whose waves issue their MFMAs at
    // raised priority, several workgroups per CU (fused q/k/v at 256 rows, 512 workgroups:
    // 40.0 against 43.9 us; q and o, 240-256 workgroups: 0.3-0.6 us slower on it). The two
    // give the same bits; only the 8-wave tile has the greedy epilogue. JV_GEMM_W8=0 / 1
    // forces one (tests, tuning).
    const char *w8env = getenv("JV_GEMM_W8");
    const size_t blocks = (w->n / plan.bn) * (size_t)jobs_or_tiles * plan.splits;
    const bool few = blocks < 2 * (size_t)std::max(1, ctx->info.compute_units);
    const bool w8 = reg && !grp && plan.bm == 64 &&
                    (greedy || (w8env ? w8env[0] != '0' : few));
    snprintf(name, sizeof name, "jv_gemm_%s_%ux%u%s%s", fmt_kernel_name(w->fmt), plan.bm, plan.bn,
             w8 ? "r8" : (reg ? "r" : ""), greedy ? "_g" : "");
    const unsigned waves = plan.bm >= 128 || w8 ? 8 : 4;
    const size_t glds = 4 * ((reg ? 0 : plan.bm) + plan.bn) / 16 * 1024;
    st = launch(ctx, name, dim3((unsigned)(w->n / plan.bn), (unsigned)jobs_or_tiles, plan.splits),
                dim3(64 * waves), glds, stream, gargs);
    if (st == JV_OK && greedy) return greedy_finish(ctx, gr, m, stream);
    if (st != JV_OK || plan.splits == 1) return st;
    const void *part = partials;
    int64_t len = (int64_t)(m * w->n);
    int sp = (int)plan.splits, ot = (int)out_type;
    void *rargs[] = {&part, &out, &len, &sp, &ot};
    return launch(ctx, "jv_reduce_splits", dim3((unsigned)((len + 255) / 256)), dim3(256), 0,
                  stream, rargs);
}

jv_status run_product(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                      const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                      jv_plan plan, jv_scratch *scratch, void *stream, GreedyArgs *gr = nullptr) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (!w) return fail(JV_ERR_INVALID, "null weight matrix");
    if (!act_ok(act)) return fail(JV_ERR_INVALID, "unknown activation type %d", (int)act);
    if (!out_ok(out_type)) return fail(JV_ERR_INVALID, "unknown output type %d", (int)out_type);
    if (!jv_plan_valid(w, m, plan))
        return fail(JV_ERR_INVALID, "plan {bm: %u, bn: %u, splits: %u} is not valid for %s [%zu, %zu] at m = %zu",
                    plan.bm, plan.bn, plan.splits, type_name(w->ggml_type).c_str(), w->n, w->k, m);
    if (x_len < m * w->k || out_len < m * w->n)
        return fail(JV_ERR_INVALID, "buffers too short: x holds %zu of %zu elements, out %zu of %zu",
                    x_len, m * w->k, out_len, m * w->n);
    if (m == 0) return JV_OK;
    if (m > (size_t)INT32_MAX) return fail(JV_ERR_INVALID, "m = %zu is too large", m);
    if (!x || !out) return fail(JV_ERR_INVALID, "null activation or output buffer");
    if (((uintptr_t)x & 15u) != 0) return fail(JV_ERR_INVALID, "activations must be 16-byte aligned");

    // Products use expert 0's rows of an expert stack (the first n rows), as the reference's
    // ungrouped kernels do (wrow = expert * n + col with expert 0, gemm.rs:463-464).
    // Small-row Q4_K, Q6_K and Q8_0 kernels: one workgroup per tile (m <= 2, up to 8 tiles
    // per compute unit); persistent workgroups that stage the activations once and stream a
    // range of tiles (wide matrices, and m > 2); split-K workgroups (below); one workgroup per
    // one or two tiles where the persistent kernel does not fit. All variants sum each output
    // element the same way, so every output row is the same for any m.
    if (plan.bm == 0 && (w->fmt == JV_FMT_Q4K || w->fmt == JV_FMT_Q6K || w->fmt == JV_FMT_Q8_0) &&
        w->n * w->experts * w->k < (1ull << 32)) {
        const bool q8 = w->fmt == JV_FMT_Q8_0, q6 = w->fmt == JV_FMT_Q6K;
        const char *fname = q8 ? "q8_0" : (q6 ? "q6k" : "q4k");
        // rows are spread over the four lane groups: ceil(m / 4) per group, the kernels' MV
        const int rpg = (int)((m + 3) / 4);
        const int mv = rpg == 1 ? 1 : (rpg == 2 ? 2 : 4);
        const int cus = std::max(1, ctx->info.compute_units);
        const int waves = q8 ? 16 : 8;
        const int ku = q8 ? 64 : 256;  // K per item
        const int xg = q6 ? 16 : 32;   // columns per activation sum
        const int U = (int)(w->k / ku);
        const int T = (int)(w->n / 16);
        const int umax = (U + waves - 1) / waves;
        const int tw = q6 || mv < 4 ? 1 : 2;  // tiles per workgroup of the per-tile kernels
        // per wave: FP16 activations [m][ku umax + 8], sums [m][ku umax / xg], for Q6_K a zero
        // row [ku umax + 8], and m range factors. The per-tile kernels reuse it for the wave's
        // tile partials (tw KB); the persistent ones add two chunks of 2 tiles x waves partials;
        // the split-K ones share one such region per workgroup, plus a flag per wave. The kernels
        // compute the same sizes.
        const size_t row = ((size_t)umax * ku + 8) * 2;
        const size_t stage = ((size_t)m * row + (size_t)m * umax * (ku / xg) * 4 + (q6 ? row : 0) +
                              (size_t)m * 4 + 15) & ~(size_t)15;
        const size_t lmax = ctx->info.lds_bytes;
        const size_t lds_persist = stage * waves + 2 * 2 * (size_t)waves * 1024;
        const size_t lds_tile = std::max(stage, (size_t)tw * 1024) * waves;
        const bool wide = T >= 8 * cus;
        // Split-K workgroups (with a scratch buffer): `waves` tiles x one of `waves` K slices
        // each, the slice staged once per workgroup (`stage` bytes of LDS). Their reduction
        // through device memory costs a few microseconds at the end, so they serve the products
        // whose per-workgroup staging is the larger cost: Q4_K and Q6_K above 8 rows, wide
        // matrices whose persistent kernel does not fit in LDS, and any K too long for the
        // per-tile kernels' LDS. Every choice below computes the same sums, so a row's bits do
        // not depend on m or on the kernel taken.
        // JV_QMV_SPLIT=0 or 1 overrides the choice where several kernels apply (tests, tuning).
        const char *force = getenv("JV_QMV_SPLIT");
        const bool fsplit = force && force[0] == '1', fnosplit = force && force[0] == '0';
        // A product given no scratch buffer (jv_matvec) whose only fitting small-row kernel is
        // split-K uses the context's own, so that its rows keep the bits of every other m.
        if (!scratch && lds_tile > lmax && !(wide && lds_persist <= lmax) && stage + 64 <= lmax)
            scratch = own_scratch(ctx);
        const bool split_ok = scratch && U >= waves && (size_t)T <= kCounterTiles && stage + 64 <= lmax;
        // Persistent workgroups stage the activations once for several tiles: they serve wide
        // matrices and, above 2 rows, any matrix (at m = 4-8 on the decode shapes 10-34% faster
        // than the per-tile kernels, whose staging per tile or tile pair dominates there).
        // JV_QMV_PERSIST=0 keeps the per-tile kernels above 2 rows (tests).
        const char *pforce = getenv("JV_QMV_PERSIST");
        const bool many = m > 2 && !(pforce && pforce[0] == '0');
        const bool persist = !(split_ok && fsplit) && (wide || many) && lds_persist <= lmax;
        const bool split = !persist && split_ok &&
                           (fsplit || lds_tile > lmax || (!fnosplit && (wide || (!q8 && m > 8))));
        const size_t lds = persist ? lds_persist : lds_tile;
        if (lds <= ctx->info.lds_bytes || split) {
            QmmParams p{};
            p.x = x;
            p.out = out;
            p.wq = w->q;
            p.M = (int32_t)m;
            p.N = (int32_t)(w->n);
            p.K = (int32_t)w->k;
            p.ldx = (int32_t)w->k;
            p.ldo = (int32_t)(w->n);
            p.act = (int32_t)act;
            p.out_type = (int32_t)out_type;
            p.splits = 1;
            void *args[] = {&p};
            char name[32];
            if (split) {
                void *partials = nullptr;
                st = scratch_reserve(scratch, (size_t)waves * m * w->n * 4, &partials);
                if (st != JV_OK) return st;
                p.part = (float *)partials;
                p.counters = (uint32_t *)scratch->buf;
                const int groups = (T + waves - 1) / waves;
                const int gp = (groups + 7) & ~7;  // the kernel's XCD mapping pads groups to 8
                snprintf(name, sizeof name, "jv_qmvs_%s_m%d", fname, mv);
                return launch(ctx, name, dim3((unsigned)(waves * gp)), dim3(64 * waves), stage + 64, stream,
                              args);
            }
            if (persist) {
                // the greedy epilogue: FP32 outputs, a variant of the same kernel
                const bool greedy = gr && out_type == JV_OUT_F32;
                snprintf(name, sizeof name, "jv_qmvp_%s_m%d%s", fname, mv, greedy ? "_g" : "");
                hipFunction_t f;
                st = get_fn(ctx, name, &f);
                if (st != JV_OK) return st;
                int per_cu = 0;
                JV_HIP(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, 64 * waves, lds));
                const int grid = std::min(T, cus * std::max(1, per_cu));
                if (greedy) {
                    st = greedy_state(ctx, m, gr);
                    if (st != JV_OK) return st;
                    p.cap = gr->cap;
                    p.amax_key = gr->key;
                    p.amax_bad = gr->bad;
                }
                st = launch(ctx, name, dim3((unsigned)grid), dim3(64 * waves), lds, stream, args);
                return st == JV_OK && greedy ? greedy_finish(ctx, gr, m, stream) : st;
            }
            snprintf(name, sizeof name, "jv_qmv_%s_t%d_m%d", fname, tw, mv);
            return launch(ctx, name, dim3((unsigned)((T + tw - 1) / tw)), dim3(64 * waves), lds, stream, args);
        }
    }
    if (pipelined_plan(w, plan))
        return launch_pipelined(ctx, x, act, m, w, out, out_type, plan, stream, nullptr, scratch, gr);
    return launch_tiles(ctx, x, act, m, w, out, out_type, scratch, plan, stream, nullptr);
}

jv_status dequant_rows(jv_ctx *ctx, const jv_qmatrix *w, size_t row0, size_t rows, void *out,
                       int f16_out, void *stream) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (!w || !out) return fail(JV_ERR_INVALID, "null matrix or output");
    if (row0 + rows > w->n * w->experts)
        return fail(JV_ERR_INVALID, "rows [%zu, %zu) are outside the %zu weight rows", row0,
                    row0 + rows, w->n * w->experts);
    if (rows == 0) return JV_OK;
    if (((uintptr_t)out & 15u) != 0) return fail(JV_ERR_INVALID, "output must be 16-byte aligned");
    DequantParams p{};
    p.wq = w->q;
    p.wh = w->h;
    p.wd = w->d;
    p.out = out;
    p.K = (int32_t)w->k;
    p.row0 = (int32_t)row0;
    p.rows = (int32_t)rows;
    p.f16_out = f16_out;
    std::string name = std::string("jv_dequant_") + fmt_kernel_name(w->fmt);
    void *args[] = {&p};
    return launch(ctx, name, dim3((unsigned)((rows + 63) / 64)), dim3(256), 0, stream, args);
}

}  // namespace

extern "C" {

// Error channel for the library's other translation units (the plan tuner); not part of the
// public header.
jv_status jv_internal_fail(jv_status st, const char *msg) { return fail(st, "%s", msg); }

jv_status jv_type_block(uint32_t ggml_type, uint32_t *elems, uint32_t *bytes) {
    uint32_t e, b;
    if (!type_block(ggml_type, &e, &b)) return fail(JV_ERR_UNSUPPORTED, "unsupported tensor type");
    if (elems) *elems = e;
    if (bytes) *bytes = b;
    return JV_OK;
}

jv_status jv_open(int device, jv_ctx **out) {
    if (!out) return fail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    int count = 0;
    JV_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return fail(JV_ERR_INVALID, "HIP device %d does not exist (%d devices)", device, count);
    JV_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    JV_HIP(hipGetDeviceProperties(&prop, device));
    if (prop.warpSize != 64 || strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(JV_ERR_UNSUPPORTED,
                    "the kernels are built for gfx950 (wave64); device %d is %s with %d-lane waves",
                    device, prop.gcnArchName, prop.warpSize);
    std::string path;
    if (const char *env = getenv("JV_CODE_OBJECT")) path = env;
    else path = library_dir() + "/jevons_qmm.hsaco";
    hipModule_t mod = nullptr;
    hipError_t e = hipModuleLoad(&mod, path.c_str());
    if (e != hipSuccess)
        return fail(JV_ERR_NO_KERNELS, "cannot load the gfx950 code object %s: %s", path.c_str(),
                    hipGetErrorString(e));
    auto *ctx = new jv_ctx();
    ctx->device = device;
    ctx->module = mod;
    ctx->info.device = device;
    ctx->info.compute_units = prop.multiProcessorCount;
    ctx->info.wave_size = prop.warpSize;
    ctx->info.lds_bytes = prop.sharedMemPerBlock;
    ctx->info.total_memory = prop.totalGlobalMem;
    snprintf(ctx->info.arch, sizeof ctx->info.arch, "%.63s", prop.gcnArchName);
    // The fixed array of jv_matmul_noalloc: its device address on this device, its tile counters
    // zeroed. A failure here is reported by jv_matmul_noalloc; the other entry points do not use it.
    void *fixed_ptr = nullptr;
    (void)jv_internal_noalloc_setup(device, kCounterBytes, &fixed_ptr);
    *out = ctx;
    return JV_OK;
}

void jv_close(jv_ctx *ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    if (ctx->pack) hipFree(ctx->pack);
    if (ctx->greedy) hipFree(ctx->greedy);
    for (void *b : ctx->retired) hipFree(b);
    jv_scratch_free(ctx->own);
    if (ctx->module) hipModuleUnload(ctx->module);
    delete ctx;
}

jv_status jv_device_info_get(jv_ctx *ctx, jv_device_info *info) {
    if (!ctx || !info) return fail(JV_ERR_INVALID, "null argument");
    *info = ctx->info;
    return JV_OK;
}

jv_status jv_sync(jv_ctx *ctx) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    JV_HIP(hipDeviceSynchronize());
    return JV_OK;
}

jv_status jv_qmatrix_upload(jv_ctx *ctx, uint32_t ggml_type, size_t n, size_t k, size_t experts,
                            const void *raw, size_t bytes, jv_qmatrix **out) {
    if (!out) return fail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    jv_fmt fmt;
    if ((st = check_upload(ggml_type, n, k, experts, bytes, &fmt)) != JV_OK) return st;
    if (!raw) return fail(JV_ERR_INVALID, "null weight bytes");
    void *tmp = nullptr;
    JV_HIP(hipMalloc(&tmp, std::max<size_t>(bytes, 16)));
    hipError_t e = hipMemcpy(tmp, raw, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(tmp);
        return fail(JV_ERR_HIP, "hipMemcpy: %s", hipGetErrorString(e));
    }
    st = build_from_device(ctx, ggml_type, fmt, n, k, experts, tmp, bytes, out);
    hipFree(tmp);
    return st;
}

jv_status jv_qmatrix_upload_device(jv_ctx *ctx, uint32_t ggml_type, size_t n, size_t k,
                                   size_t experts, const void *raw_dev, size_t bytes,
                                   jv_qmatrix **out) {
    if (!out) return fail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    jv_fmt fmt;
    if ((st = check_upload(ggml_type, n, k, experts, bytes, &fmt)) != JV_OK) return st;
    if (!raw_dev) return fail(JV_ERR_INVALID, "null weight bytes");
    return build_from_device(ctx, ggml_type, fmt, n, k, experts, raw_dev, bytes, out);
}

jv_status jv_qmatrix_from_packed(jv_ctx *ctx, uint32_t ggml_type, size_t n, size_t k,
                                 size_t experts, const uint32_t *q, size_t nq, const uint32_t *h,
                                 size_t nh, const uint32_t *s, size_t ns, const float *d,
                                 size_t nd, jv_qmatrix **out) {
    if (!out) return fail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    uint32_t block, size;
    if (!type_block(ggml_type, &block, &size)) return fail(JV_ERR_UNSUPPORTED, "unsupported type");
    const std::string kind = type_name(ggml_type);
    size_t wq = 0, wh = 0, ws = 0, wd = 0;  // quant::packed_words (quant.rs:127-135)
    switch (ggml_type) {
    case JV_GGML_Q4K: wq = 36; break;
    case JV_GGML_Q6K: wq = 32; wh = 16; ws = 4; wd = 1; break;
    case JV_GGML_Q5_0: wq = 4; wh = 1; wd = 1; break;
    case JV_GGML_Q8_0: wq = 8; wd = 1; break;
    default: return fail(JV_ERR_UNSUPPORTED, "%s weights are not supported", kind.c_str());
    }
    const size_t blocks = experts * n * k / block;
    if (k % 64 != 0 || n % 64 != 0 || k % block != 0 || nq != blocks * wq || nh != blocks * wh ||
        ns != blocks * ws || nd != blocks * wd)
        return fail(JV_ERR_INVALID, "%s [%zux%zu, %zu] has an unsupported shape", kind.c_str(),
                    experts, n, k);
    if ((nq && !q) || (nh && !h) || (ns && !s) || (nd && !d))
        return fail(JV_ERR_INVALID, "null packed region");
    // Rebuild the GGML blocks (the inverse of quant::pack, quant.rs:156-193).
    std::vector<uint8_t> raw(blocks * size);
    for (size_t b = 0; b < blocks; ++b) {
        uint8_t *o = raw.data() + b * size;
        if (wd) {
            float v = d[b];
            if (f16_bits_to_f32(f32_to_f16_bits(v)) != v && !(std::isnan(v)))
                return fail(JV_ERR_INVALID, "%s packed scale %zu (%g) is not an FP16 value",
                            kind.c_str(), b, (double)v);
        }
        switch (ggml_type) {
        case JV_GGML_Q4K: memcpy(o, q + 36 * b, 144); break;
        case JV_GGML_Q6K:
            memcpy(o, q + 32 * b, 128);
            memcpy(o + 128, h + 16 * b, 64);
            memcpy(o + 192, s + 4 * b, 16);
            put_f16(raw, b * size + 208, d[b]);
            break;
        case JV_GGML_Q5_0:
            put_f16(raw, b * size, d[b]);
            memcpy(o + 2, h + b, 4);
            memcpy(o + 6, q + 4 * b, 16);
            break;
        case JV_GGML_Q8_0:
            put_f16(raw, b * size, d[b]);
            memcpy(o + 2, q + 8 * b, 32);
            break;
        }
    }
    return jv_qmatrix_upload(ctx, ggml_type, n, k, experts, raw.data(), raw.size(), out);
}

jv_status jv_qmatrix_f16_view(jv_ctx *ctx, size_t n, size_t k, const void *dev_words, size_t words,
                              jv_qmatrix **out) {
    if (!out) return fail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    if (!ctx) return fail(JV_ERR_INVALID, "null context");
    if (k % 64 != 0 || n % 64 != 0 || words != n * k / 2 || n > (size_t)INT32_MAX)
        return fail(JV_ERR_INVALID, "F16 [%zu, %zu] has an unsupported shape", n, k);
    if (!dev_words || ((uintptr_t)dev_words & 15u) != 0)
        return fail(JV_ERR_INVALID, "F16 weights must be a 16-byte aligned device buffer");
    auto *w = new jv_qmatrix();
    w->ctx = ctx;
    w->ggml_type = JV_GGML_F16;
    w->fmt = JV_FMT_F16;
    w->n = n;
    w->k = k;
    w->experts = 1;
    w->q = (const uint8_t *)dev_words;
    w->h = w->q;
    w->d = w->q;
    w->bytes = n * k * 2;
    *out = w;
    return JV_OK;
}

void jv_qmatrix_free(jv_qmatrix *w) {
    if (!w) return;
    if (w->base) {
        hipSetDevice(w->ctx->device);
        hipFree(w->base);
    }
    delete w;
}

size_t jv_qmatrix_bytes(const jv_qmatrix *w) { return w ? w->bytes : 0; }

jv_status jv_qmatrix_shape(const jv_qmatrix *w, uint32_t *fmt, size_t *n, size_t *k,
                           size_t *experts) {
    if (!w) return fail(JV_ERR_INVALID, "null matrix");
    if (fmt) *fmt = (uint32_t)w->fmt;
    if (n) *n = w->n;
    if (k) *k = w->k;
    if (experts) *experts = w->experts;
    return JV_OK;
}

// Plan::heuristic (gemm.rs:987-1004), tile_n (:968-971) and choose_splits (:1032-1038).
jv_plan jv_plan_heuristic(const jv_qmatrix *w, size_t m, int row_invariant, size_t groups_target) {
    if (!w) return jv_plan{0, 0, 0};
    const uint32_t bm = m <= 32 ? 32 : 64;
    const uint32_t bn = w->n % 128 == 0 ? 128 : 64;
    if (row_invariant) return jv_plan{bm, bn, 1};
    if (m <= 2) return jv_plan{0, bn, 1};
    const size_t base = (w->n / bn) * ((m + bm - 1) / bm);
    const size_t steps = w->k / 64;
    uint32_t splits = 1;
    while (splits < 16 && base * splits < groups_target && steps / (splits * 2) >= 4) splits *= 2;
    return jv_plan{bm, bn, splits};
}

// gfx950 choice: the small-row kernel up to 16 rows; otherwise the row tile that covers m with
// the least padding, then the widest column tile that still gives every compute unit a
// workgroup, then (outside prefill) split-K until the grid fills the device.
// Products outside prefill may split K (their rows may then differ by plan, as the reference
// allows for canvas products, tune.rs:170-173). Long K (8192 and more) takes the 256- or
// 128-row tile and enough slices to give every compute unit a workgroup: each weight is then
// decoded once per 256 rows and the activations are read by half as many column tiles (down
// projection, K = 15360 at m = 256: 67 us on 256 x 128 / 8 against 100 us on whole-K 64 x 64).
// Otherwise a tile whose workgroups fill less than three quarters of the device doubles its
// slices until they fill it (k and v projections, 2048 x 3840 at m = 256: 64 x 64 / 2, 26
// against 29 us). Slices stay whole 256-element blocks, at least four of them.
static jv_plan canvas_split(const jv_qmatrix *w, size_t m, jv_plan p, size_t cus) {
    if (w->k >= 8192 && m >= 128 && w->n % 128 == 0) p = m >= 192 ? jv_plan{256, 128, 1} : jv_plan{128, 128, 1};
    const size_t wgs = (w->n / p.bn) * ((m + p.bm - 1) / p.bm);
    if (w->k >= 8192 || wgs * 4 < cus * 3) {
        uint32_t s = 1;
        while (wgs * s < cus && w->k / 256 / (2 * s) >= 4 && block_slices(w, 2 * s)) s *= 2;
        p.splits = s;
    }
    return p;
}

jv_plan jv_plan_auto(const jv_qmatrix *w, size_t m, int row_invariant) {
    if (!w) return jv_plan{0, 0, 0};
    // The small-row kernel keeps a row's bits independent of m but not equal to the tile
    // kernels' bits, so row-invariant (prefill) products always take tiles (gemm.rs:989-994).
    if (m <= 16 && !row_invariant) return jv_plan{0, 64, 1};
    const size_t cus = w->ctx ? (size_t)std::max(1, w->ctx->info.compute_units) : 256;
    const size_t cols = w->n;
    // Pipelined tiles (whole K, so row invariant): 256 x 128 when that gives about one workgroup
    // per compute unit (each weight decoded once per 256 rows); otherwise 64 x 64, which keeps
    // more compute units busy on narrow matrices and wastes the least on a few rows (at m = 32
    // of the Q6_K vocabulary projection it beats the 32-row generic tiles by 1.6x). A few rows
    // of a narrow matrix outside prefill keep the generic tiles, whose split-K fills the device.
    const size_t tiles64 = (cols / 64) * ((m + 63) / 64);
    if (w->k % 256 == 0 && (m >= 48 || row_invariant || tiles64 >= cus)) {
        jv_plan p{0, 0, 1};
        // 256 x 128 from 192 rows (at most a quarter of its rows padding), 128 x 128 above 64
        // rows, each only while its workgroups still fill the device (gate_up at m = 128:
        // 55 us on 128 x 128 against 69 us on 256 x 128 and 60 us on 64 x 64)
        if (cols % 128 == 0 && m >= 192 && ((m + 255) / 256) * (cols / 128) * 16 >= cus * 15)
            p = jv_plan{256, 128, 1};
        else if (cols % 128 == 0 && m > 64 && ((m + 127) / 128) * (cols / 128) * 16 >= cus * 15)
            p = jv_plan{128, 128, 1};
        // up to 32 rows: half a 64-row tile would be padding (Q6_K vocabulary projection at
        // m = 32: 235 us against 281 us on 64 x 64; Q8_0 4096 x 4096: 25 against 29 us)
        else if (cols % 64 == 0 && m <= 32 && reg_format(w))
            p = jv_plan{32, 64, 1};
        else if (cols % 64 == 0)
            p = jv_plan{64, 64, 1};
        if (p.bm != 0) return row_invariant ? p : canvas_split(w, m, p, cus);
    }
    const uint32_t bm = m <= 32 ? 32 : (m <= 64 ? 64 : 128);
    const size_t mtiles = (m + bm - 1) / bm;
    uint32_t bn = 64;
    for (uint32_t c : {256u, 128u}) {
        if (w->n % c == 0 && (w->n / c) * mtiles >= cus) {
            bn = c;
            break;
        }
    }
    uint32_t splits = 1;
    if (!row_invariant) {
        const size_t base = (w->n / bn) * mtiles;
        const size_t units = w->k / (size_t)fmt_unit(w->fmt);
        while (splits < 16 && base * splits < cus && units / (splits * 2) >= 4) splits *= 2;
    }
    return jv_plan{bm, bn, splits};
}

// Plan::valid_for (gemm.rs:1006-1015); gfx950 also accepts 256-column tiles.
int jv_plan_valid(const jv_qmatrix *w, size_t m, jv_plan p) {
    if (!w) return 0;
    if (p.bm == 0) return m <= 16 && p.splits == 1;
    // gfx950 tile: 256 rows x 128 columns, split-K only in whole 256-element blocks
    if (p.bm == 256) return p.bn == 128 && w->n % 128 == 0 && block_slices(w, p.splits) && p.splits <= 16;
    const bool bm_ok = p.bm == 32 || p.bm == 64 || p.bm == 128;
    const bool bn_ok = p.bn == 64 || p.bn == 128 || p.bn == 256;
    return bm_ok && bn_ok && w->n % p.bn == 0 && p.splits >= 1 && p.splits <= 16 &&
           w->k / 64 >= p.splits;
}

jv_status jv_scratch_new(jv_ctx *ctx, jv_scratch **out) {
    if (!ctx || !out) return fail(JV_ERR_INVALID, "null argument");
    auto *s = new jv_scratch();
    s->ctx = ctx;
    *out = s;
    return JV_OK;
}

void jv_scratch_free(jv_scratch *s) {
    if (!s) return;
    if (s->buf || !s->retired.empty()) {
        hipSetDevice(s->ctx->device);
        if (s->buf) hipFree(s->buf);
        for (void *b : s->retired) hipFree(b);
    }
    delete s;
}

jv_status jv_matmul(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                    const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                    jv_scratch *scratch, void *stream) {
    if (!w) return fail(JV_ERR_INVALID, "null weight matrix");
    if (!ctx) return fail(JV_ERR_INVALID, "null context");
    // a split-K plan given no scratch buffer stages its partials in the context's own
    const jv_plan plan = jv_plan_auto(w, m, 0);
    if (plan.splits > 1 && !scratch) scratch = own_scratch(ctx);
    return run_product(ctx, x, act, x_len, m, w, out, out_type, out_len, plan, scratch, stream);
}

jv_status jv_matmul_noalloc(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                            const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                            void *stream) {
    if (!ctx) return fail(JV_ERR_INVALID, "null context");
    if (!w) return fail(JV_ERR_INVALID, "null weight matrix");
    hipError_t e = hipSuccess;
    void *ptr = jv_internal_noalloc_ptr(ctx->device, &e);
    if (!ptr)
        return fail(JV_ERR_HIP, "the fixed scratch array is not set up on device %d: %s", ctx->device,
                    hipGetErrorString(e));
    // jv_matmul with a scratch buffer that is the fixed array: same plan, kernels and bits; the
    // buffer never grows (a product needing more is rejected before any launch)
    jv_scratch fixed;
    fixed.ctx = ctx;
    fixed.buf = ptr;
    fixed.bytes = JV_NOALLOC_SCRATCH_BYTES;
    fixed.fixed = true;
    // A split-K tile plan whose activations and partials would not fit in the array runs with
    // whole K instead (same tile, no partials).
    jv_plan plan = jv_plan_auto(w, m, 0);
    if (plan.bm != 0 && plan.splits > 1) {
        const size_t rows = (m + plan.bm - 1) / plan.bm * plan.bm;
        const size_t need = align_up(rows * w->k * 2 + rows * 4, 256) + (size_t)plan.splits * m * w->n * 4;
        if (need > JV_NOALLOC_SCRATCH_BYTES - kCounterBytes) plan.splits = 1;
    }
    return run_product(ctx, x, act, x_len, m, w, out, out_type, out_len, plan, &fixed, stream);
}

jv_status jv_matmul_plan(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                         const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                         jv_scratch *scratch, jv_plan plan, void *stream) {
    return run_product(ctx, x, act, x_len, m, w, out, out_type, out_len, plan, scratch, stream);
}

jv_status jv_matvec(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                    const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                    void *stream) {
    if (m > 16) return fail(JV_ERR_INVALID, "matvec handles at most 16 rows, got %zu", m);
    return run_product(ctx, x, act, x_len, m, w, out, out_type, out_len, jv_plan{0, 64, 1},
                       nullptr, stream);
}

jv_status jv_matmul_split(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                          const jv_qmatrix *w, void *out, jv_out out_type, size_t out_len,
                          uint32_t bm, uint32_t bn, uint32_t splits, jv_scratch *scratch,
                          void *stream) {
    if (bm == 0) return fail(JV_ERR_INVALID, "matmul_split needs a row tile (bm > 0)");
    return run_product(ctx, x, act, x_len, m, w, out, out_type, out_len,
                       jv_plan{bm, bn, splits}, scratch, stream);
}

jv_status jv_group_routes(jv_ctx *ctx, const uint32_t *ids, size_t assignments, size_t experts,
                          uint32_t bm, uint32_t *sorted, uint32_t *offsets, uint32_t *jobs,
                          size_t jobs_len, void *stream) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (experts == 0 || experts > 1024)
        return fail(JV_ERR_INVALID, "grouping handles 1 to 1024 experts, got %zu", experts);
    if (bm == 0) return fail(JV_ERR_INVALID, "row tile bm must be positive");
    if (assignments > (size_t)UINT32_MAX) return fail(JV_ERR_INVALID, "too many routes");
    if (jobs_len < 1 + 2 * ((assignments + bm - 1) / bm + experts))
        return fail(JV_ERR_INVALID, "jobs buffer of %zu words is too small", jobs_len);
    if ((assignments && (!ids || !sorted)) || !offsets || !jobs)
        return fail(JV_ERR_INVALID, "null buffer");
    uint32_t a = (uint32_t)assignments, e = (uint32_t)experts, b = bm;
    void *args[] = {&ids, &a, &e, &b, &sorted, &offsets, &jobs};
    return launch(ctx, "jv_group_routes", dim3(1), dim3(1024), 0, stream, args);
}

namespace {
// Checks shared by the grouped products (gemm.rs:1172, :1285).
jv_status check_grouped(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, const jv_qmatrix *w,
                        const jv_groups *g, void *out, size_t out_len) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (!w || !g) return fail(JV_ERR_INVALID, "null matrix or groups");
    if (act != JV_ACT_F16 && act != JV_ACT_BF16 && act != JV_ACT_F32)
        return fail(JV_ERR_INVALID, "unknown activation type");
    if (out_len < g->rows * w->n)
        return fail(JV_ERR_INVALID, "output holds %zu values, grouped product writes %zu", out_len,
                    g->rows * w->n);
    if (g->in_div == 0) return fail(JV_ERR_INVALID, "in_div must be positive");
    if (x_len < (g->rows + g->in_div - 1) / g->in_div * w->k)
        return fail(JV_ERR_INVALID, "activations hold %zu values, need %zu", x_len,
                    (g->rows + g->in_div - 1) / g->in_div * w->k);
    if (g->rows && (!x || !out || !g->ids || !g->offsets || !g->jobs))
        return fail(JV_ERR_INVALID, "null buffer");
    if (((uintptr_t)x & 15u) != 0) return fail(JV_ERR_INVALID, "activations must be 16-byte aligned");
    if (g->max_jobs > 65535) return fail(JV_ERR_INVALID, "max_jobs %zu is too large", g->max_jobs);
    return JV_OK;
}
}  // namespace

jv_status jv_matmul_grouped(jv_ctx *ctx, const void *x, jv_act act, size_t x_len,
                            const jv_qmatrix *w, const jv_groups *g, void *out, jv_out out_type,
                            size_t out_len, uint32_t bm, uint32_t bn, uint32_t splits,
                            jv_scratch *scratch, void *stream) {
    jv_status st = check_grouped(ctx, x, act, x_len, w, g, out, out_len);
    if (st != JV_OK) return st;
    if (bm != 16 && bm != 32 && bm != 64 && bm != 128)
        return fail(JV_ERR_INVALID, "grouped row tile %u is not 16, 32, 64 or 128", bm);
    if ((bn != 64 && bn != 128 && bn != 256) || w->n % bn != 0)
        return fail(JV_ERR_INVALID, "n = %zu is not a multiple of the column tile %u", w->n, bn);
    if (splits < 1 || splits > 16 || w->k / 64 < splits)
        return fail(JV_ERR_INVALID, "splits = %u is out of range", splits);
    if (g->rows == 0 || g->max_jobs == 0) return JV_OK;
    GroupArgs ga{g->ids, g->offsets, g->jobs, g->max_jobs, g->in_div, bm};
    // 64 x 64 and 128 x 128 jobs on the pipelined tiles (same bits as the generic tiles) while
    // the per-job packed activations stay within 1 GiB
    if (bm != 256 && splits == 1 && pipelined_plan(w, jv_plan{bm, bn, splits}) &&
        g->max_jobs * bm * w->k * 2 <= (1ull << 30))
        return launch_pipelined(ctx, x, act, g->rows, w, out, out_type, jv_plan{bm, bn, splits},
                                stream, &ga);
    return launch_tiles(ctx, x, act, g->rows, w, out, out_type, scratch, jv_plan{bm, bn, splits},
                        stream, &ga);
}

jv_status jv_matvec_grouped(jv_ctx *ctx, const void *x, jv_act act, size_t x_len,
                            const jv_qmatrix *w, const jv_groups *g, void *out, jv_out out_type,
                            size_t out_len, uint32_t mr, void *stream) {
    jv_status st = check_grouped(ctx, x, act, x_len, w, g, out, out_len);
    if (st != JV_OK) return st;
    if (mr == 0 || mr > 16) return fail(JV_ERR_INVALID, "matvec_grouped handles 1 to 16 rows per job");
    if (g->rows == 0 || g->max_jobs == 0) return JV_OK;
    // Q4_K, Q6_K and Q8_0 jobs run the small-row per-tile kernel in grouped mode (grid y = job),
    // which streams each job's expert weights as the decode GEMV does. Jobs of up to 8 rows go
    // through in one pass (rows spread over the lane groups); larger ones in chunks of 2, so
    // the LDS holds at most 8 rows. 128 experts [1408, 2816], 8 / 32 tokens x top-8: jobs of
    // up to 4 rows (the reference's SMALL_GROUP_ROWS) 27 / 67 us against 46 / 84 us on the
    // generic grouped tiles (and 31 / 87 us in 2-row chunks); mr = 16 30 / 81 us against 89 /
    // 185 us. JV_QMVG=0 takes the generic tiles.
    const char *genv = getenv("JV_QMVG");
    if ((w->fmt == JV_FMT_Q4K || w->fmt == JV_FMT_Q6K || w->fmt == JV_FMT_Q8_0) &&
        w->n * w->experts * w->k < (1ull << 32) && !(genv && genv[0] == '0')) {
        const bool q8 = w->fmt == JV_FMT_Q8_0, q6 = w->fmt == JV_FMT_Q6K;
        const int waves = 4;  // as the jv_qmvg_* kernels are built
        const int ku = q8 ? 64 : 256;  // K per item
        const int xg = q6 ? 16 : 32;   // columns per activation sum
        const int U = (int)(w->k / ku);
        const int umax = (U + waves - 1) / waves;
        // per wave, as the kernel computes it: FP16 activations [mv][ku umax + 8], sums
        // [mv][ku umax / xg], a zero row for Q6_K, mv range factors; at least the 1 KB of the
        // tile partial
        const size_t mv = mr <= 8 ? mr : 2;  // rows per pass
        const size_t row = ((size_t)umax * ku + 8) * 2;
        const size_t stage = (mv * row + mv * umax * (ku / xg) * 4 + (q6 ? row : 0) + mv * 4 + 15) & ~(size_t)15;
        const size_t lds = std::max(stage, (size_t)1024) * waves;
        if (lds <= ctx->info.lds_bytes) {
            QmmParams p{};
            p.x = x;
            p.out = out;
            p.wq = w->q;
            p.M = (int32_t)mr;
            p.N = (int32_t)(w->n);
            p.K = (int32_t)w->k;
            p.ldx = (int32_t)w->k;
            p.ldo = (int32_t)(w->n);
            p.act = (int32_t)act;
            p.out_type = (int32_t)out_type;
            p.splits = 1;
            p.ids = g->ids;
            p.offsets = g->offsets;
            p.jobs = g->jobs;
            p.grouped = 1;
            p.in_div = (int32_t)g->in_div;
            p.rows_cap = (int32_t)mr;
            void *args[] = {&p};
            char name[32];
            snprintf(name, sizeof name, "jv_qmvg_%s_%s", q8 ? "q8_0" : (q6 ? "q6k" : "q4k"),
                     mr <= 4 ? "m1" : (mr <= 8 ? "m2" : "c2"));
            return launch(ctx, name, dim3((unsigned)(w->n / 16), (unsigned)g->max_jobs), dim3(64 * waves),
                          lds, stream, args);
        }
    }
    GroupArgs ga{g->ids, g->offsets, g->jobs, g->max_jobs, g->in_div, mr};
    return launch_tiles(ctx, x, act, g->rows, w, out, out_type, nullptr, jv_plan{16, 64, 1}, stream,
                        &ga);
}

// crates/jevons-burn/src/kernels.rs:52-97 with the row-invariant plan rule of :16-31.
jv_status jv_f16_matmul(jv_ctx *ctx, const void *x, size_t m, size_t k, const void *weight,
                        size_t n, float *out, void *stream) {
    if (!ctx) return fail(JV_ERR_INVALID, "null context");
    if (k % 64 != 0 || n % 64 != 0)
        return fail(JV_ERR_INVALID, "f16 matmul weight shape (N and K must be multiples of 64)");
    jv_qmatrix view;
    view.ctx = ctx;
    view.ggml_type = JV_GGML_F16;
    view.fmt = JV_FMT_F16;
    view.n = n;
    view.k = k;
    view.q = view.h = view.d = (const uint8_t *)weight;
    if (!weight || ((uintptr_t)weight & 15u) != 0)
        return fail(JV_ERR_INVALID, "F16 weights must be a 16-byte aligned device buffer");
    uint32_t bm, bn;
    if (m <= 32) {
        if (k > 8192) { bm = 128; bn = 128; }
        else if (n >= 16384 && n < 65536 && n % 128 == 0) { bm = 64; bn = 128; }
        else { bm = 32; bn = 64; }
    } else if (m <= 64) {
        bm = 64; bn = n % 128 == 0 ? 128 : 64;
    } else {
        bm = 128; bn = n % 128 == 0 ? 128 : 64;
    }
    return run_product(ctx, x, JV_ACT_F16, m * k, m, &view, out, JV_OUT_F32, m * n,
                       jv_plan{bm, bn, 1}, nullptr, stream);
}

jv_status jv_argmax_rows(jv_ctx *ctx, const float *logits, size_t rows, size_t n, int32_t *index,
                         jv_scratch *scratch, void *stream) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (rows == 0) return JV_OK;
    if (!index || (n && !logits)) return fail(JV_ERR_INVALID, "null buffer");
    if (!scratch) return fail(JV_ERR_INVALID, "argmax needs a scratch buffer");
    if (n > (size_t)INT32_MAX || rows > 65535)
        return fail(JV_ERR_INVALID, "argmax of %zu rows x %zu is too large", rows, n);
    // Rows that are 16-byte aligned take 1-4 float4 loads per thread per chunk of 1024-4096
    // values, the chunk halved until the grid holds about 1024 workgroups; others scalar loads.
    const bool vec = n % 4 == 0 && ((uintptr_t)logits & 15u) == 0;
    int chunk = vec ? 4096 : 2048;
    while (vec && chunk > 1024 && rows * ((n + chunk - 1) / chunk) < 1024) chunk /= 2;
    int chunks = (int)((n + chunk - 1) / chunk);
    const size_t need = std::max<size_t>(rows * (size_t)chunks * 8, 16);
    void *partials = nullptr;
    st = scratch_reserve(scratch, need, &partials);
    if (st != JV_OK) return st;
    float *pval = (float *)partials;
    int *pidx = (int *)((uint8_t *)partials + rows * (size_t)chunks * 4);
    if (chunks > 0) {
        int64_t nn = (int64_t)n;
        int ch = chunk, v = vec ? 1 : 0;
        void *a1[] = {&logits, &nn, &ch, &v, &pval, &pidx};
        st = launch(ctx, "jv_argmax_partial", dim3((unsigned)chunks, (unsigned)rows), dim3(256), 0,
                    stream, a1);
        if (st != JV_OK) return st;
    }
    return launch_argmax_final(ctx, pval, pidx, chunks, rows, index, stream);
}

jv_status jv_matmul_argmax(jv_ctx *ctx, const void *x, jv_act act, size_t x_len, size_t m,
                           const jv_qmatrix *w, float *out, size_t out_len, float cap, int32_t *index,
                           jv_scratch *scratch, void *stream) {
    if (!ctx) return fail(JV_ERR_INVALID, "null context");
    if (!w) return fail(JV_ERR_INVALID, "null weight matrix");
    if (!(cap >= 0.f) || !std::isfinite(cap))
        return fail(JV_ERR_INVALID, "softcap %g must be 0 (none) or positive", (double)cap);
    if (!index && m > 0) return fail(JV_ERR_INVALID, "null index buffer");
    if (!scratch) return fail(JV_ERR_INVALID, "argmax needs a scratch buffer");
    if (m > 65535 || w->n > (size_t)INT32_MAX)
        return fail(JV_ERR_INVALID, "argmax of %zu rows x %zu is too large", m, w->n);
    // jv_matmul's plan; its small-row persistent kernels and 32 x 64 tiles have a variant with
    // the greedy epilogue, and any other kernel is followed by the soft cap and jv_argmax_rows
    const jv_plan plan = jv_plan_auto(w, m, 0);
    GreedyArgs gr;
    gr.cap = cap;
    gr.index = index;
    jv_status st = run_product(ctx, x, act, x_len, m, w, out, JV_OUT_F32, out_len, plan, scratch, stream, &gr);
    if (st != JV_OK || m == 0 || gr.done) return st;
    if (cap > 0.f) {
        st = jv_softcap_logits(ctx, out, m * w->n, cap, stream);
        if (st != JV_OK) return st;
    }
    return jv_argmax_rows(ctx, out, m, w->n, index, scratch, stream);
}

jv_status jv_softcap_logits(jv_ctx *ctx, float *x, size_t len, float cap, void *stream) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (!(cap > 0.f) || !std::isfinite(cap)) return fail(JV_ERR_INVALID, "softcap %g must be positive", (double)cap);
    if (len == 0) return JV_OK;
    if (!x) return fail(JV_ERR_INVALID, "null buffer");
    int64_t n = (int64_t)len;
    void *args[] = {&x, &n, &cap};
    return launch(ctx, "jv_softcap", dim3((unsigned)((len + 1023) / 1024)), dim3(256), 0, stream, args);
}

jv_status jv_pick_logits(jv_ctx *ctx, const void *x, jv_act act, size_t x_len,
                         const jv_qmatrix *table, const uint32_t *pairs, size_t count, float *out,
                         size_t out_len, float cap, void *stream) {
    jv_status st = use_device(ctx);
    if (st != JV_OK) return st;
    if (!table) return fail(JV_ERR_INVALID, "null table");
    if (act != JV_ACT_F16 && act != JV_ACT_BF16 && act != JV_ACT_F32)
        return fail(JV_ERR_INVALID, "unknown activation type");
    if (!(cap > 0.f) || !std::isfinite(cap)) return fail(JV_ERR_INVALID, "softcap %g must be positive", (double)cap);
    if (out_len < count) return fail(JV_ERR_INVALID, "output holds %zu values, need %zu", out_len, count);
    const size_t d = table->k;
    if (x_len % d != 0) return fail(JV_ERR_INVALID, "activations (%zu) are not rows of %zu", x_len, d);
    if (count == 0) return JV_OK;
    if (!x || !pairs || !out) return fail(JV_ERR_INVALID, "null buffer");
    if (count > (size_t)INT32_MAX || table->n * table->experts > (size_t)INT32_MAX ||
        x_len / d > (size_t)INT32_MAX)
        return fail(JV_ERR_INVALID, "pick_logits shape is too large");
    PickParams p{};
    p.x = x;
    p.pairs = pairs;
    p.wq = table->q;
    p.wh = table->h;
    p.wd = table->d;
    p.out = out;
    p.d = (int32_t)d;
    p.act = (int32_t)act;
    p.count = (int32_t)count;
    p.x_rows = (int32_t)(x_len / d);
    p.n = (int32_t)(table->n * table->experts);
    p.cap = cap;
    char name[40];
    snprintf(name, sizeof name, "jv_pick_logits_%s", fmt_kernel_name(table->fmt));
    void *args[] = {&p};
    return launch(ctx, name, dim3((unsigned)count), dim3(256), 0, stream, args);
}

jv_status jv_dequant_rows_f32(jv_ctx *ctx, const jv_qmatrix *w, size_t row0, size_t rows,
                              float *out, void *stream) {
    return dequant_rows(ctx, w, row0, rows, out, 0, stream);
}

jv_status jv_dequant_rows_f16(jv_ctx *ctx, const jv_qmatrix *w, size_t row0, size_t rows,
                              uint16_t *out, void *stream) {
    return dequant_rows(ctx, w, row0, rows, out, 1, stream);
}

const char *jv_last_error(void) { return g_error.c_str(); }

}  // extern "C"

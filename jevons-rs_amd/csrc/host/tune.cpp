// Launch-plan tuner and its on-disk table: the counterpart of
// crates/jevons-gemma4-diffusion/src/gpu/tune.rs, built on this library's public C ABI.
//
// Plans are keyed by (weight format, n, k, row bucket, row invariance) for dense products and by
// (format, n, k, experts, row bucket) for expert-grouped ones. A bucket b serves row counts in
// (b/2, b] (tune.rs:73-76). Measured plans replace the fallback only when at least 5% faster
// (tune.rs:556-566), and row-invariant lookups only accept whole-K tile plans (tune.rs:485-487),
// so tuning never changes a prefill row's bits. The fallback is this library's own plan rule
// (jv_plan_auto); the reference falls back to Plan::heuristic, which is tuned for its own GPU.
//
// Table text format (tune.rs:358-444): a profile line that must match this device, then
//   dense <fmt> <n> <k> <bucket> <row_invariant 0|1> <bm> <bn> <splits>
//   grouped <fmt> <n> <k> <experts> <bucket> <bm> <bn>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "jevons_qmm.h"

namespace {

constexpr int kTuneVersion = 1;

struct DenseKey {
    uint32_t fmt;
    size_t n, k, bucket;
    int row_invariant;
    bool operator<(const DenseKey &o) const {
        return std::tie(fmt, n, k, row_invariant, bucket) < std::tie(o.fmt, o.n, o.k, o.row_invariant, o.bucket);
    }
};

struct GroupKey {
    uint32_t fmt;
    size_t n, k, experts, bucket;
    bool operator<(const GroupKey &o) const {
        return std::tie(fmt, n, k, experts, bucket) < std::tie(o.fmt, o.n, o.k, o.experts, o.bucket);
    }
};

struct GroupPlan {
    uint32_t bm, bn;
};

size_t next_pow2(size_t v) {
    size_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

}  // namespace

struct jv_tuner {
    jv_ctx *ctx = nullptr;  // null: table only (no measurement)
    std::string key;
    std::string path;  // empty: nothing is stored
    std::map<DenseKey, jv_plan> dense;
    std::map<GroupKey, GroupPlan> grouped;
};

// The library's error channel (jv_last_error), defined in jevons_qmm.cpp.
extern "C" jv_status jv_internal_fail(jv_status st, const char *msg);

namespace {

jv_status tfail(jv_status st, const char *msg) { return jv_internal_fail(st, msg); }

// Profile line (tune.rs:64-75): what the measured plans depend on.
std::string profile_key(const jv_device_info &info) {
    std::string arch = info.arch;
    const size_t colon = arch.find(':');
    if (colon != std::string::npos) arch = arch.substr(0, colon);
    char buf[256];
    snprintf(buf, sizeof buf, "v%d device=%d cus=%d wave=%d lds=%zu arch=%s", kTuneVersion, info.device,
             info.compute_units, info.wave_size, info.lds_bytes, arch.c_str());
    return buf;
}

void load_table(jv_tuner *t) {
    if (t->path.empty()) return;
    std::ifstream in(t->path);
    if (!in) return;
    std::string line;
    if (!std::getline(in, line) || line != t->key) return;  // another device or version
    while (std::getline(in, line)) {
        std::istringstream ls(line);
        std::string kind;
        ls >> kind;
        if (kind == "dense") {
            size_t fmt, n, k, b, ri, bm, bn, sp;
            if (ls >> fmt >> n >> k >> b >> ri >> bm >> bn >> sp)
                t->dense[DenseKey{(uint32_t)fmt, n, k, b, ri == 1}] = jv_plan{(uint32_t)bm, (uint32_t)bn, (uint32_t)sp};
        } else if (kind == "grouped") {
            size_t fmt, n, k, e, b, bm, bn;
            if (ls >> fmt >> n >> k >> e >> b >> bm >> bn)
                t->grouped[GroupKey{(uint32_t)fmt, n, k, e, b}] = GroupPlan{(uint32_t)bm, (uint32_t)bn};
        }
    }
}

// Seconds per run of `run` (tune.rs:568-594): one untimed run, then the best of three batches
// sized to take at least ~2 ms, timed with events on the null stream.
template <class Run>
double time_runs(Run run, jv_status *st) {
    *st = run();
    if (*st != JV_OK) return 0.0;
    hipDeviceSynchronize();
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    hipEventRecord(a, nullptr);
    *st = run();
    hipEventRecord(b, nullptr);
    hipEventSynchronize(b);
    float once_ms = 0.f;
    hipEventElapsedTime(&once_ms, a, b);
    const int reps = std::clamp((int)std::ceil(2.0 / std::max(1e-3, (double)once_ms)), 1, 32);
    double best = 1e30;
    for (int i = 0; i < 3 && *st == JV_OK; ++i) {
        hipEventRecord(a, nullptr);
        for (int r = 0; r < reps && *st == JV_OK; ++r) *st = run();
        hipEventRecord(b, nullptr);
        hipEventSynchronize(b);
        float ms = 0.f;
        hipEventElapsedTime(&ms, a, b);
        best = std::min(best, (double)ms * 1e-3 / reps);
    }
    hipEventDestroy(a);
    hipEventDestroy(b);
    return best;
}

// Candidate plans (tune.rs:499-530, with the gfx950 tiles added): the small-row kernel for
// m <= 16 when rows may vary in bits, every reference tile that fits the rows, split-K only
// when row invariance is not asked for, and the pipelined tiles (256 x 128 also split in
// whole 256-element blocks outside prefill).
std::vector<jv_plan> dense_candidates(const jv_qmatrix *w, size_t m, int row_invariant) {
    uint32_t fmt;
    size_t n, k, experts;
    jv_qmatrix_shape(w, &fmt, &n, &k, &experts);
    std::vector<jv_plan> out;
    if (!row_invariant && m <= 16) out.push_back(jv_plan{0, n % 128 == 0 ? 128u : 64u, 1});
    const size_t steps = k / 64;
    for (uint32_t bm : {32u, 64u, 128u}) {
        if (bm > 32 && bm > m) continue;
        for (uint32_t bn : {64u, 128u, 256u}) {
            if (n % bn != 0 || (bm == 128 && bn == 64)) continue;
            for (uint32_t sp : {1u, 2u, 4u, 8u}) {
                if (sp > 1 && (row_invariant || steps / sp < 4 || (bm == 128 && sp > 4))) continue;
                out.push_back(jv_plan{bm, bn, sp});
            }
        }
    }
    for (jv_plan p : {jv_plan{256, 128, 1}, jv_plan{128, 128, 1}, jv_plan{64, 64, 1}, jv_plan{256, 128, 2},
                      jv_plan{256, 128, 4}, jv_plan{256, 128, 8}})
        if ((p.splits == 1 || !row_invariant) && jv_plan_valid(w, m, p) &&
            std::none_of(out.begin(), out.end(), [&](const jv_plan &q) {
                return q.bm == p.bm && q.bn == p.bn && q.splits == p.splits;
            }))
            out.push_back(p);
    out.erase(std::remove_if(out.begin(), out.end(), [&](const jv_plan &p) { return !jv_plan_valid(w, m, p); }),
              out.end());
    return out;
}

bool same_plan(const jv_plan &a, const jv_plan &b) { return a.bm == b.bm && a.bn == b.bn && a.splits == b.splits; }

}  // namespace

extern "C" {

size_t jv_tune_bucket(size_t m) { return std::max<size_t>(next_pow2(std::max<size_t>(m, 1)), 4); }

size_t jv_tune_buckets(size_t min, size_t max, size_t *out, size_t cap) {
    size_t count = 0;
    const size_t top = jv_tune_bucket(std::max<size_t>(max, 1));
    for (size_t b = min; b > 0 && b <= top && b <= 1024; b *= 2) {
        if (out && count < cap) out[count] = b;
        ++count;
    }
    return count;
}

int jv_tune_pick(const double *times, const uint32_t *ids, size_t n, uint32_t baseline) {
    if (n == 0 || !times || !ids) return -1;
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (times[i] < times[best]) best = i;
    for (size_t i = 0; i < n; ++i)
        if (ids[i] == baseline && times[best] > times[i] * (1.0 - 0.05)) return (int)i;
    return (int)best;
}

jv_status jv_tuner_new(jv_ctx *ctx, const char *path, jv_tuner **out) {
    if (!out) return tfail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    if (!ctx) return tfail(JV_ERR_INVALID, "null context");
    jv_device_info info{};
    jv_status st = jv_device_info_get(ctx, &info);
    if (st != JV_OK) return st;
    auto *t = new jv_tuner();
    t->ctx = ctx;
    t->key = profile_key(info);
    t->path = path ? path : "";
    load_table(t);
    *out = t;
    return JV_OK;
}

jv_status jv_tuner_open_table(const char *profile, const char *path, jv_tuner **out) {
    if (!out || !profile) return tfail(JV_ERR_INVALID, "null argument");
    auto *t = new jv_tuner();
    t->key = profile;
    t->path = path ? path : "";
    load_table(t);
    *out = t;
    return JV_OK;
}

void jv_tuner_free(jv_tuner *t) { delete t; }

const char *jv_tuner_profile(const jv_tuner *t) { return t ? t->key.c_str() : ""; }

size_t jv_tuner_entries(const jv_tuner *t) { return t ? t->dense.size() + t->grouped.size() : 0; }

int jv_tuner_lookup_dense(const jv_tuner *t, uint32_t fmt, size_t n, size_t k, size_t m,
                          int row_invariant, jv_plan *plan) {
    if (!t || !plan) return 0;
    auto it = t->dense.find(DenseKey{fmt, n, k, jv_tune_bucket(m), row_invariant ? 1 : 0});
    if (it == t->dense.end()) return 0;
    *plan = it->second;
    return 1;
}

void jv_tuner_insert_dense(jv_tuner *t, uint32_t fmt, size_t n, size_t k, size_t bucket,
                           int row_invariant, jv_plan plan) {
    if (t) t->dense[DenseKey{fmt, n, k, bucket, row_invariant ? 1 : 0}] = plan;
}

void jv_tuner_insert_grouped(jv_tuner *t, uint32_t fmt, size_t n, size_t k, size_t experts,
                             size_t bucket, uint32_t bm, uint32_t bn) {
    if (t) t->grouped[GroupKey{fmt, n, k, experts, bucket}] = GroupPlan{bm, bn};
}

jv_plan jv_tuner_dense(const jv_tuner *t, const jv_qmatrix *w, size_t m, int row_invariant) {
    uint32_t fmt = 0;
    size_t n = 0, k = 0, experts = 0;
    if (t && jv_qmatrix_shape(w, &fmt, &n, &k, &experts) == JV_OK) {
        jv_plan p;
        if (jv_tuner_lookup_dense(t, fmt, n, k, m, row_invariant, &p) && jv_plan_valid(w, m, p) &&
            (!row_invariant || (p.bm > 0 && p.splits == 1)))
            return p;
    }
    return jv_plan_auto(w, m, row_invariant);
}

jv_status jv_tuner_grouped(const jv_tuner *t, const jv_qmatrix *w, size_t rows, uint32_t *bm,
                           uint32_t *bn) {
    if (!bm || !bn) return tfail(JV_ERR_INVALID, "null output");
    uint32_t fmt;
    size_t n, k, experts;
    jv_status st = jv_qmatrix_shape(w, &fmt, &n, &k, &experts);
    if (st != JV_OK) return st;
    *bm = 32;  // GroupPlan::heuristic (tune.rs:106-111)
    *bn = n % 128 == 0 ? 128 : 64;
    if (t) {
        auto it = t->grouped.find(GroupKey{fmt, n, k, experts, jv_tune_bucket(rows)});
        if (it != t->grouped.end() && n % it->second.bn == 0) {
            *bm = it->second.bm;
            *bn = it->second.bn;
        }
    }
    return JV_OK;
}

jv_status jv_tuner_tune_dense(jv_tuner *t, const jv_qmatrix *const *ws, size_t nws, size_t m,
                              int row_invariant, const void *x, jv_act act, size_t x_len,
                              void *out, size_t out_len, jv_scratch *scratch, int *added) {
    if (added) *added = 0;
    if (!t || !t->ctx) return tfail(JV_ERR_INVALID, "tuner has no device");
    if (!ws || nws == 0 || !ws[0]) return tfail(JV_ERR_INVALID, "no matrices");
    uint32_t fmt;
    size_t n, k, experts;
    jv_status st = jv_qmatrix_shape(ws[0], &fmt, &n, &k, &experts);
    if (st != JV_OK) return st;
    const DenseKey key{fmt, n, k, m, row_invariant ? 1 : 0};
    if (t->dense.count(key) || x_len < m * k || out_len < m * n || k % 64 != 0) return JV_OK;
    const jv_plan baseline = jv_plan_auto(ws[0], m, row_invariant);
    std::vector<jv_plan> cands = dense_candidates(ws[0], m, row_invariant);
    if (std::none_of(cands.begin(), cands.end(), [&](const jv_plan &p) { return same_plan(p, baseline); }))
        cands.push_back(baseline);
    std::vector<double> times;
    std::vector<uint32_t> ids;
    uint32_t base_id = 0;
    for (size_t c = 0; c < cands.size(); ++c) {
        const jv_plan p = cands[c];
        double s = time_runs([&] {
            for (size_t i = 0; i < nws; ++i) {
                jv_status r = jv_matmul_plan(t->ctx, x, act, x_len, m, ws[i], out, JV_OUT_F32, out_len,
                                             scratch, p, nullptr);
                if (r != JV_OK) return r;
            }
            return JV_OK;
        }, &st);
        if (st != JV_OK) return st;
        times.push_back(s);
        ids.push_back((uint32_t)c);
        if (same_plan(p, baseline)) base_id = (uint32_t)c;
    }
    const int pick = jv_tune_pick(times.data(), ids.data(), times.size(), base_id);
    if (pick >= 0) {
        t->dense[key] = cands[(size_t)pick];
        if (added) *added = 1;
    }
    return JV_OK;
}

jv_status jv_tuner_tune_grouped(jv_tuner *t, const jv_qmatrix *const *ws, size_t nws, size_t rows,
                                size_t top_k, const void *x, jv_act act, size_t x_len, void *out,
                                size_t out_len, uint32_t *route_ids, size_t route_capacity,
                                uint32_t *sorted, uint32_t *offsets, uint32_t *jobs, size_t jobs_len,
                                jv_scratch *scratch, int *added) {
    if (added) *added = 0;
    if (!t || !t->ctx) return tfail(JV_ERR_INVALID, "tuner has no device");
    if (!ws || nws == 0 || !ws[0] || top_k == 0) return tfail(JV_ERR_INVALID, "no matrices");
    uint32_t fmt;
    size_t n, k, experts;
    jv_status st = jv_qmatrix_shape(ws[0], &fmt, &n, &k, &experts);
    if (st != JV_OK) return st;
    const GroupKey key{fmt, n, k, experts, rows};
    const size_t a = rows * top_k;
    if (t->grouped.count(key) || route_capacity < a || x_len < a * k || out_len < a * n) return JV_OK;
    // synthetic balanced routing (tune.rs:320-324): each token picks top_k distinct experts
    std::vector<uint32_t> host(route_capacity);
    for (size_t i = 0; i < route_capacity; ++i)
        host[i] = (uint32_t)(((i / top_k) * 7 + (i % top_k) * 13) % experts);
    if (hipMemcpy(route_ids, host.data(), route_capacity * 4, hipMemcpyHostToDevice) != hipSuccess)
        return tfail(JV_ERR_HIP, "route upload failed");
    std::vector<GroupPlan> cands;
    for (uint32_t bm : {32u, 64u})
        for (uint32_t bn : {64u, 128u})
            if (n % bn == 0) cands.push_back(GroupPlan{bm, bn});
    const GroupPlan baseline{32, n % 128 == 0 ? 128u : 64u};
    std::vector<double> times;
    std::vector<uint32_t> ids;
    std::vector<GroupPlan> timed;
    uint32_t base_id = 0;
    for (size_t c = 0; c < cands.size(); ++c) {
        const GroupPlan p = cands[c];
        const size_t max_jobs = (a + p.bm - 1) / p.bm + experts;
        if (jobs_len < 1 + 2 * max_jobs) continue;
        st = jv_group_routes(t->ctx, route_ids, a, experts, p.bm, sorted, offsets, jobs, jobs_len, nullptr);
        if (st != JV_OK) return st;
        const jv_groups g{sorted, offsets, jobs, max_jobs, 1, a};
        double s = time_runs([&] {
            for (size_t i = 0; i < nws; ++i) {
                jv_status r = jv_matmul_grouped(t->ctx, x, act, x_len, ws[i], &g, out, JV_OUT_F32, out_len,
                                                p.bm, p.bn, 1, scratch, nullptr);
                if (r != JV_OK) return r;
            }
            return JV_OK;
        }, &st);
        if (st != JV_OK) return st;
        if (p.bm == baseline.bm && p.bn == baseline.bn) base_id = (uint32_t)times.size();
        ids.push_back((uint32_t)times.size());
        times.push_back(s);
        timed.push_back(p);
    }
    const int pick = jv_tune_pick(times.data(), ids.data(), times.size(), base_id);
    if (pick >= 0) {
        t->grouped[key] = timed[(size_t)pick];
        if (added) *added = 1;
    }
    return JV_OK;
}

jv_status jv_tuner_save(const jv_tuner *t) {
    if (!t) return tfail(JV_ERR_INVALID, "null tuner");
    if (t->path.empty()) return JV_OK;
    std::string outs = t->key + "\n";
    char buf[256];
    for (const auto &e : t->dense) {
        snprintf(buf, sizeof buf, "dense %u %zu %zu %zu %d %u %u %u\n", e.first.fmt, e.first.n, e.first.k,
                 e.first.bucket, e.first.row_invariant, e.second.bm, e.second.bn, e.second.splits);
        outs += buf;
    }
    for (const auto &e : t->grouped) {
        snprintf(buf, sizeof buf, "grouped %u %zu %zu %zu %zu %u %u\n", e.first.fmt, e.first.n, e.first.k,
                 e.first.experts, e.first.bucket, e.second.bm, e.second.bn);
        outs += buf;
    }
    const std::string tmp = t->path + ".tmp";
    {
        std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
        if (!f || !(f << outs)) return tfail(JV_ERR_INVALID, "cannot write the plan table");
    }
    if (std::rename(tmp.c_str(), t->path.c_str()) != 0) return tfail(JV_ERR_INVALID, "cannot store the plan table");
    return JV_OK;
}

}  // extern "C"

"""Pins the CPU oracle before anything is compared against it.

Each restated function is checked against the reference's own known-answer tests
(crates/jevons-formats/src/quant.rs:195-237, crates/jevons-core/src/model.rs:221-234), against a
library routine where one exists (numpy/torch float conversions, numpy matmul), or against
hand-built blocks whose decoded values follow from the block layout alone, so that a wrong
index, shift, sign or dropped term fails one of them.
"""
import json
import os
import struct

import numpy as np
import pytest
import torch


def f16_bytes(v: float) -> bytes:
    return np.float16(v).tobytes()


# ---------------------------------------------------------------- f16 / bf16 conversions

def test_f16_to_f32_matches_numpy_for_all_65536_patterns(oracle):
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = pats.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(p)) for p in pats], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rounds_to_nearest_even_like_numpy(oracle):
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-3),
        rng.standard_normal(20000).astype(np.float32) * np.float32(300.0),
        (rng.random(5000).astype(np.float32) * np.float32(1e-6)),  # subnormal range
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24,
                  2.0 ** -25, 2.0 ** -25 * 1.0000001, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                  np.inf, -np.inf], dtype=np.float32),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_bf16_conversions_match_torch(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(6)
    vals = rng.standard_normal(5000).astype(np.float32) * np.float32(50.0)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.jvo_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)
    back = np.array([L.jvo_bf16_to_f32(int(h)) for h in want], dtype=np.float32)
    assert np.array_equal(back, torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------- type table

def test_type_table_matches_gguf_block_sizes(oracle):
    # gguf.rs:134-144
    assert oracle.type_block(0) == (1, 4)
    assert oracle.type_block(1) == (1, 2)
    assert oracle.type_block(6) == (32, 22)
    assert oracle.type_block(8) == (32, 34)
    assert oracle.type_block(12) == (256, 144)
    assert oracle.type_block(14) == (256, 210)
    for other in (2, 3, 7, 10, 11, 13, 15, 30):
        assert oracle.type_block(other) is None
    assert oracle.packed_words(12) == (36, 0, 0, 0)
    assert oracle.packed_words(14) == (32, 16, 4, 1)
    assert oracle.packed_words(6) == (4, 1, 0, 1)
    assert oracle.packed_words(8) == (8, 0, 0, 1)


# ---------------------------------------------------------------- reference KATs
# Vectors of the reference's own unit tests, kept in tests/golden/reference_kats.json
# (written by tests/golden/make_kats.py).

KATS = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                   "reference_kats.json")))


def test_q4k_decodes_scale_high_bits_for_upper_groups(oracle):
    kat = KATS["q4k_scale_min"]  # quant.rs:199-208
    q = bytes(kat["scale_bytes"])
    for j, pair in kat["pairs"].items():
        assert oracle.q4k_scale_min(int(j), q) == tuple(pair)


def test_q8_0_and_q5_0_dequantize_signed_values(oracle):
    for name, type_id in (("q8_0", oracle.Q8_0), ("q5_0", oracle.Q5_0)):  # quant.rs:210-226
        kat = KATS[name]
        out = oracle.dequantize(type_id, np.frombuffer(bytes.fromhex(kat["block_hex"]), np.uint8))
        for i, v in kat["expect"].items():
            assert out[int(i)] == v, (name, i)


def test_packing_splits_quants_and_scales_without_changing_values(oracle):
    kat = KATS["pack_q8_0"]  # quant.rs:228-237
    q8 = bytes.fromhex(kat["block_hex"])
    q, h, s, d = oracle.pack(oracle.Q8_0, np.frombuffer(q8, np.uint8))
    assert len(q) == kat["q_words"] and list(d) == kat["d"]
    assert q[0] == kat["q0"]
    with pytest.raises(oracle.OracleError):
        oracle.pack(oracle.Q8_0, np.frombuffer(q8[:33], np.uint8))


def test_greedy_takes_the_first_argmax_with_its_stable_probability(oracle):
    for case in KATS["greedy"]["cases"]:  # crates/jevons-core/src/model.rs:221-234
        logits = np.array([float(v) for v in case["logits"]], np.float32)
        if case.get("error"):
            with pytest.raises(oracle.OracleError):
                oracle.greedy(logits)
            continue
        tok, conf = oracle.greedy(logits)
        assert tok == case["index"]
        if "prob" in case:
            assert abs(conf - case["prob"]) < case["prob_tol"]
    with pytest.raises(oracle.OracleError):
        oracle.greedy(np.array([], np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.greedy(np.array([1.0, np.nan], np.float32))


def test_dequantize_rejects_bad_sizes_and_types(oracle):
    with pytest.raises(oracle.OracleError, match="size mismatch"):
        oracle.dequantize(oracle.Q4K, np.zeros(143, np.uint8), 256)
    with pytest.raises(oracle.OracleError, match="size mismatch"):
        oracle.dequantize(oracle.Q4K, np.zeros(144, np.uint8), 255)
    with pytest.raises(oracle.OracleError, match="unsupported"):
        oracle.dequantize(2, np.zeros(18, np.uint8), 32)
    with pytest.raises(oracle.OracleError, match="no GPU block layout"):
        oracle.pack(oracle.F16, np.zeros(4, np.uint8))


# ---------------------------------------------------------------- hand-built Q4_K blocks

def q4k_block(d, dmin, scales12, qs128):
    return np.frombuffer(f16_bytes(d) + f16_bytes(dmin) + bytes(scales12) + bytes(qs128), np.uint8)


def test_q4k_unit_scales_decode_to_the_raw_nibbles(oracle):
    # scales 0..3 = 1 (bytes 0..3), mins 0 (bytes 4..7), scales 4..7 = 1 (low nibbles of 8..11)
    scales = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    qs = [(i * 7 + 3) & 0xFF for i in range(128)]
    w = oracle.dequantize(oracle.Q4K, q4k_block(1.0, 0.0, scales, qs))
    for p in range(4):
        for l in range(32):
            b = qs[32 * p + l]
            assert w[64 * p + l] == (b & 15)
            assert w[64 * p + 32 + l] == (b >> 4)


def test_q4k_single_nibble_lands_at_its_element_with_its_sub_block_scale(oracle):
    # KAT scale bytes give (scale, min) = (1,5) (2,6) (3,7) (4,8) (50,33) (36,51) (22,5) (8,23):
    # j=5: (0x34&15)|((0x82>>6)<<4) = 36, (0x34>>4)|((0xc6>>6)<<4) = 51; j=6: 6|16 = 22, 5|0 = 5
    scales = [0xc1, 0x82, 0x43, 0x04, 0x85, 0xc6, 0x07, 0x48, 0x12, 0x34, 0x56, 0x78]
    pairs = [(1, 5), (2, 6), (3, 7), (4, 8), (50, 33), (36, 51), (22, 5), (8, 23)]
    assert [oracle.q4k_scale_min(j, bytes(scales)) for j in range(8)] == pairs
    d, dmin = 0.5, 0.25
    for p, l, lo, hi in [(0, 0, 3, 0), (1, 17, 0, 9), (2, 31, 15, 15), (3, 5, 1, 2)]:
        qs = [0] * 128
        qs[32 * p + l] = lo | (hi << 4)
        w = oracle.dequantize(oracle.Q4K, q4k_block(d, dmin, scales, qs))
        want = np.array([-dmin * pairs[e // 32][1] for e in range(256)], np.float32)
        want[64 * p + l] = d * pairs[2 * p][0] * lo - dmin * pairs[2 * p][1]
        want[64 * p + 32 + l] = d * pairs[2 * p + 1][0] * hi - dmin * pairs[2 * p + 1][1]
        assert np.array_equal(w, want), (p, l)


def test_q4k_matches_a_vectorised_restatement_on_random_blocks(oracle):
    rng = np.random.default_rng(7)
    nb = 64
    raw = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    raw[:, 0:2] = np.frombuffer(np.abs(rng.standard_normal(nb)).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
    raw[:, 2:4] = np.frombuffer(np.abs(rng.standard_normal(nb)).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
    got = oracle.dequantize(oracle.Q4K, raw).reshape(nb, 256)
    # vectorised over blocks, following the GGML block_q4_K layout description:
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dm = raw[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = raw[:, 4:16].astype(np.uint32)
    sc = np.zeros((nb, 8), np.uint32)
    mn = np.zeros((nb, 8), np.uint32)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = raw[:, 16:].reshape(nb, 4, 32)
    nib = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float32)
    want = (d[:, None, None] * sc[:, :, None].astype(np.float32)) * nib - \
        (dm[:, None] * mn.astype(np.float32))[:, :, None]
    assert np.array_equal(got, want.reshape(nb, 256).astype(np.float32))


# ---------------------------------------------------------------- hand-built Q6_K blocks

def q6k_block(ql, qh, sc, d):
    return np.frombuffer(bytes(ql) + bytes(qh) + bytes([s & 0xFF for s in sc]) + f16_bytes(d), np.uint8)


def q6_element_position(e):
    """(ql byte, ql shift, qh byte, qh shift) holding element e of a Q6_K block."""
    n, r = divmod(e, 128)
    i, l = divmod(r, 32)
    ql = 64 * n + l + (32 if i in (1, 3) else 0)
    return ql, (4 if i >= 2 else 0), 32 * n + l, 2 * i


def test_q6k_zero_point_and_sign_of_scales(oracle):
    # q6 = 32 everywhere: low nibble 0, high bits 2 -> every element decodes to 0
    ql = [0] * 128
    qh = [0b10101010] * 64
    w = oracle.dequantize(oracle.Q6K, q6k_block(ql, qh, [1] * 16, 1.0))
    assert np.array_equal(w, np.zeros(256, np.float32))
    # one element at a time with distinct scales: w = d * sc[e // 16] * (q6 - 32). The high
    # bits take every value, three of them unlike the background's 2, so an element read from
    # the wrong qh bits (or a neighbour given this one's) decodes wrong.
    scales = [(-1) ** g * (g + 1) for g in range(16)]
    for q6 in (45, 61, 13, 29):  # low nibble 13, high bits 2, 3, 0, 1
        for e in [0, 15, 16, 33, 70, 95, 127, 128, 161, 200, 255]:
            ql = [0] * 128
            qh = [0b10101010] * 64
            b, sh, hb, hsh = q6_element_position(e)
            ql[b] |= (q6 & 15) << sh
            qh[hb] = (qh[hb] & ~(3 << hsh)) | ((q6 >> 4) << hsh)
            w = oracle.dequantize(oracle.Q6K, q6k_block(ql, qh, scales, 0.5))
            want = np.zeros(256, np.float32)
            want[e] = 0.5 * scales[e // 16] * (q6 - 32)
            assert np.array_equal(w, want), (q6, e)


def test_q5_0_high_bits_follow_qh_bit_order(oracle):
    for j in range(32):
        blk = bytearray(22)
        blk[0:2] = f16_bytes(2.0)
        blk[2:6] = struct.pack("<I", 1 << j)
        w = oracle.dequantize(oracle.Q5_0, np.frombuffer(bytes(blk), np.uint8))
        want = np.full(32, -32.0, np.float32)
        want[j] = 0.0  # (16 - 16) * 2
        assert np.array_equal(w, want), j


# ---------------------------------------------------------------- packing invariant

@pytest.mark.parametrize("tid", [8, 14, 6, 12])
def test_pack_keeps_values(oracle, tid):
    rng = np.random.default_rng(tid)
    e, b = oracle.type_block(tid)
    nb = 12
    raw = rng.integers(0, 256, size=(nb, b), dtype=np.uint8)
    # keep the f16 scales finite
    off = {8: 0, 6: 0, 12: 0, 14: 208}[tid]
    raw[:, off:off + 2] = np.frombuffer(np.float16(0.75).tobytes(), np.uint8)
    if tid == 12:
        raw[:, 2:4] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    q, h, s, d = oracle.pack(tid, raw)
    wq, wh, ws, wd = oracle.packed_words(tid)
    assert (len(q), len(h), len(s), len(d)) == (nb * wq, nb * wh, nb * ws, nb * wd)
    qb = q.view(np.uint8).reshape(nb, -1)
    if tid == 12:
        assert np.array_equal(qb, raw)
    elif tid == 14:
        assert np.array_equal(qb, raw[:, :128])
        assert np.array_equal(h.view(np.uint8).reshape(nb, -1), raw[:, 128:192])
        assert np.array_equal(s.view(np.uint8).reshape(nb, -1), raw[:, 192:208])
        assert np.all(d == 0.75)
    elif tid == 8:
        assert np.array_equal(qb, raw[:, 2:])
        assert np.all(d == 0.75)
    else:
        assert np.array_equal(qb, raw[:, 6:])
        assert np.array_equal(h.view(np.uint8).reshape(nb, -1), raw[:, 2:6])


# ---------------------------------------------------------------- f64 matmul

def test_matmul_f64_matches_numpy_and_a_hand_example(oracle):
    x = np.array([[1.0, 2.0, 3.0]], np.float32)
    w = np.array([[1.0, 0.0, -1.0], [0.5, 0.25, 0.125]], np.float32)
    assert np.array_equal(oracle.matmul_f64(x, w), np.array([[-2.0, 1.375]]))
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 300)).astype(np.float32)
    w = rng.standard_normal((70, 300)).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(oracle.matmul_f64(x, w), want, rtol=1e-12, atol=1e-12)


def test_cpu_baseline_agrees_with_the_f64_oracle(oracle):
    rng = np.random.default_rng(9)
    n, k, m = 64, 512, 3
    raw = oracle.Rng(11).recipe_q8_0(n * k // 32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = oracle.dequantize(oracle.Q8_0, raw).reshape(n, k)
    want = oracle.matmul_f64(x, w)
    for threads in (1, 0):
        got = oracle.cpu_dequant_matmul(oracle.Q8_0, raw, n, k, x, threads=threads)
        assert oracle.normalized_error(got, want) < 1e-5


# ---------------------------------------------------------------- fixture generator

def test_xorshift_fixture_generator(oracle):
    # gpu/tests.rs:11-23, restated with Python integers
    s = 11
    r = oracle.Rng(11)
    for _ in range(1000):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        want = np.float32(np.float32(s >> 40) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0))
        assert r.next() == want


# ------------------------------------------------------------------ expert grouping

def test_group_routes_hand_example(oracle):
    """ops::group (gpu/ops.rs:522-587) on a small route list: experts in order, each expert's
    assignments in assignment order, one (expert, start) job per bm-row tile."""
    ids = np.array([2, 0, 2, 1, 0, 2, 2], np.uint32)
    sorted_, offsets, jobs = oracle.group_routes(ids, 3, 2)
    assert sorted_.tolist() == [1, 4, 3, 0, 2, 5, 6]
    assert offsets.tolist() == [0, 2, 3, 7]
    assert jobs[0] == 4
    assert jobs[1:9].tolist() == [0, 0, 1, 2, 2, 3, 2, 5]


@pytest.mark.parametrize("experts,bm,a", [(4, 32, 42), (8, 16, 100), (16, 64, 7), (5, 1, 30)])
def test_group_routes_invariants(oracle, experts, bm, a):
    """Brute-force properties of the grouping: every routed assignment appears once, experts
    are contiguous and ascending, order is stable within an expert, the jobs tile every expert's
    range with bm rows (the coverage check of gpu/tests.rs:340-357), ids >= experts are dropped."""
    rng = np.random.default_rng(experts * 1000 + bm)
    ids = rng.integers(0, experts + 1, a).astype(np.uint32)  # value `experts` is not routed
    sorted_, offsets, jobs = oracle.group_routes(ids, experts, bm)
    routed = [i for i in range(a) if ids[i] < experts]
    assert sorted(sorted_.tolist()) == routed
    for e in range(experts):
        seg = sorted_[offsets[e]:offsets[e + 1]].tolist()
        assert seg == [i for i in range(a) if ids[i] == e]
    covered = 0
    for j in range(jobs[0]):
        e, start = int(jobs[1 + 2 * j]), int(jobs[2 + 2 * j])
        assert offsets[e] <= start < offsets[e + 1] and (start - offsets[e]) % bm == 0
        covered += min(int(offsets[e + 1]) - start, bm)
    assert covered == len(routed)
    assert jobs[0] == sum((int(offsets[e + 1] - offsets[e]) + bm - 1) // bm for e in range(experts))


def test_grouped_product_reference(oracle):
    """The f64 grouped product equals per-assignment products of the expert's rows."""
    rng = np.random.default_rng(5)
    experts, n, k, in_div = 3, 4, 8, 2
    w = rng.standard_normal((experts * n, k)).astype(np.float32)
    x = rng.standard_normal((3, k)).astype(np.float32)
    ids = np.array([1, 0, 2, 2, 0, 1])
    got = oracle.grouped_product_f64(x, w, ids, in_div, n)
    for a, e in enumerate(ids):
        want = x[a // in_div].astype(np.float64) @ w[e * n:(e + 1) * n].astype(np.float64).T
        assert np.allclose(got[a], want, rtol=0, atol=1e-12)


def test_softcap_is_a_smooth_clamp(oracle):
    """cap tanh(v / cap) (gpu/ops.rs:750-758): odd, zero at zero, identity to first order for
    |v| << cap, bounded by cap and approaching it."""
    cap = 30.0
    v = np.array([-1e6, -90.0, -1e-3, 0.0, 1e-3, 15.0, 90.0, 1e6])
    got = oracle.softcap(v, cap)
    assert got[3] == 0.0
    assert np.allclose(got, -oracle.softcap(-v, cap), rtol=0, atol=0)
    assert abs(got[4] - 1e-3) < 1e-12 and np.all(np.abs(got) <= cap)
    assert cap - got[-1] < 1e-9 and abs(got[5] - 30.0 * np.tanh(0.5)) < 1e-12


def test_pick_logits_is_the_softcapped_product_at_each_pair(oracle):
    """pick_logits (gpu/ops.rs:589-634): the logit of pair (row, token) is softcap(x[row] .
    E[token]). A hand example, and every pair of a non-square case against the f64 product,
    so that swapped pair roles or a transposed table fail."""
    x = np.array([[1.0, 2.0]], np.float32)
    table = np.array([[3.0, 4.0], [5.0, 6.0], [7.0, 8.0]], np.float32)
    got = oracle.pick_logits_f64(x, table, np.array([[0, 1], [0, 2]]), 1e9)
    assert np.allclose(got, [17.0, 23.0], rtol=1e-12, atol=0)
    assert abs(oracle.pick_logits_f64(x, table, np.array([[0, 0]]), 10.0)[0] - 10.0 * np.tanh(1.1)) < 1e-12
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, 8)).astype(np.float32)
    table = rng.standard_normal((5, 8)).astype(np.float32)
    pairs = np.array([[0, 4], [2, 1], [1, 1], [2, 4], [0, 0]])
    full = oracle.softcap(oracle.matmul_f64(x, table), 30.0)
    got = oracle.pick_logits_f64(x, table, pairs, 30.0)
    assert np.allclose(got, [full[r, t] for r, t in pairs], rtol=0, atol=1e-12)

"""GPU parity of the gfx950 products against the CPU oracle (quant.rs decode + f64 matmul).

Bars: dequantized weights bit-exact (FP32 decode == quant::dequantize; FP16 tile == round to
nearest even of it); outputs within 1e-3 of max|f64 oracle| (the reference's own bar is 2e-3,
crates/jevons-gemma4-diffusion/src/gpu/tests.rs:427-480); plans without split-K bitwise
identical to each other (spec R8).
"""
import numpy as np
import pytest
import torch

import jevons_qmm as jq
import oracle as O
from helpers import activations, err, f16_tensor, oracle_product, say
from jevons_qmm import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
FORMATS = [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0), ("q5_0", jq.Q5_0), ("f16", jq.F16)]


@pytest.fixture(scope="module")
def gpu():
    g = jq.Gpu(0)
    say("device", g.info.arch.decode(), "CUs", g.info.compute_units, "LDS", g.info.lds_bytes)
    yield g


def make_matrix(gpu, type_id, n, k, seed, raw=None):
    if raw is None:
        raw = synth.weights(type_id, seed, n, k)
    if type_id == jq.F16:
        t = torch.from_numpy(raw.view(np.float16).reshape(n, k).copy()).cuda()
        return jq.QMatrix.f16_view(gpu, n, k, t), raw
    return jq.QMatrix.upload(gpu, type_id, n, k, 1, raw), raw


# ------------------------------------------------------------------ exact weight decode

@pytest.mark.parametrize("name,type_id", FORMATS)
def test_device_decode_is_bit_exact(gpu, name, type_id):
    n, k = 128, 1024
    say("decode", name, n, k)
    w, raw = make_matrix(gpu, type_id, n, k, seed=3)
    want = O.dequantize(type_id, raw).reshape(n, k)
    got = jq.dequant_rows(gpu, w, 0, n).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    tile = jq.dequant_rows(gpu, w, 0, n, f16=True).cpu().numpy()
    assert np.array_equal(tile.view(np.uint16), want.astype(np.float16).view(np.uint16))
    # a row range that starts inside the matrix
    part = jq.dequant_rows(gpu, w, 37, 50).cpu().numpy()
    assert np.array_equal(part.view(np.uint32), want[37:87].view(np.uint32))


# FP16 block scales beyond the synthetic ones (bit patterns): signed zeros, the smallest and
# largest subnormals, +-1, the largest finite values, infinities, NaN, and an ordinary value
_EXTREME_F16 = np.array([0x0000, 0x8000, 0x0001, 0x83FF, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x7C00,
                         0xFC00, 0x7E00, 0x1234], np.uint16)
# finite ones whose decoded weights stay inside the FP16 range for every format (|d| <= 8)
_FINITE_F16 = np.array([0x0000, 0x8000, 0x0001, 0x83FF, 0x0400, 0x3C00, 0xBC00, 0xB800, 0xC800], np.uint16)
_SCALE_FIELDS = {jq.Q4K: (144, (0, 2)), jq.Q6K: (210, (208,)), jq.Q8_0: (34, (0,)), jq.Q5_0: (22, (0,))}


def _with_scales(type_id, raw, patterns, seed):
    """Every block's FP16 scale fields (Q4_K: d and dmin) set to patterns drawn from `patterns`;
    Q6_K's int8 sub-block scales over their whole range (-128 included)."""
    rng = np.random.default_rng(seed)
    bsize, offs = _SCALE_FIELDS[type_id]
    blocks = raw.reshape(-1, bsize).copy()
    for o in offs:
        pick = patterns[rng.integers(0, patterns.size, blocks.shape[0])]
        blocks[:, o:o + 2] = pick.view(np.uint8).reshape(-1, 2)
    if type_id == jq.Q6K:
        blocks[:, 192:208] = rng.integers(0, 256, size=(blocks.shape[0], 16), dtype=np.uint8)
    return blocks.reshape(-1)


def _same_bits_nan_as_nan(got, want, uint):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), "NaN positions differ"
    bad = np.argwhere(got[~nan].view(uint) != want[~nan].view(uint))
    assert bad.size == 0, f"{bad.size} elements differ"


@pytest.mark.parametrize("name,type_id", [f for f in FORMATS if f[1] != jq.F16])
def test_device_decode_of_extreme_scales(gpu, name, type_id):
    """Block scales of every FP16 class: the device's FP32 decode equals quant.rs's arithmetic
    bit for bit (NaN where it is NaN: payloads are not compared), and the FP16 tile is its
    round to nearest even (overflowing to infinity where the FP32 value is beyond FP16)."""
    n, k = 64, 1024
    raw = _with_scales(type_id, synth.weights(type_id, 60, n, k), _EXTREME_F16, 61)
    w = jq.QMatrix.upload(gpu, type_id, n, k, 1, raw)
    want = O.dequantize(type_id, raw).reshape(n, k)
    assert np.isnan(want).any() and np.isinf(want).any()
    _same_bits_nan_as_nan(jq.dequant_rows(gpu, w, 0, n).cpu().numpy(), want, np.uint32)
    _same_bits_nan_as_nan(jq.dequant_rows(gpu, w, 0, n, f16=True).cpu().numpy(),
                          want.astype(np.float16), np.uint16)


@pytest.mark.parametrize("name,type_id", [f for f in FORMATS if f[1] != jq.F16])
def test_products_with_extreme_finite_scales(gpu, name, type_id):
    """Zero, negative and subnormal block scales through the products: every tiled plan's
    on-chip tile is the reference's FP16 tile (identity activations), and the small-row and
    tiled products match the f64 oracle."""
    n, k = 128, 512
    raw = _with_scales(type_id, synth.weights(type_id, 62, n, k), _FINITE_F16, 63)
    w = jq.QMatrix.upload(gpu, type_id, n, k, 1, raw)
    dense = O.dequantize(type_id, raw).reshape(n, k)
    assert np.isfinite(dense).all() and (dense < 0).any()
    tile = dense.astype(np.float16).astype(np.float32)
    assert np.isfinite(tile).all()
    x = torch.eye(k, dtype=torch.float16, device="cuda")
    plans = [jq.Plan(32, 64, 1), jq.Plan(32, 128, 1), jq.Plan(64, 64, 1), jq.Plan(128, 128, 1),
             jq.Plan(256, 128, 1)]
    for plan in [pl for pl in plans if pl.valid_for(w, k)]:
        out = torch.empty((k, n), dtype=torch.float32, device="cuda")
        jq.matmul_plan(gpu, x, k, w, out, None, plan)
        got = out.cpu().numpy()
        want = tile.T.copy() + np.float32(0.0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), plan
    scratch = jq.SplitScratch(gpu)
    for m in (1, 4, 16, 40):
        xb, xv = activations("bf16", synth.normal_rows(64 + m, m, k))
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, xb, m, w, out, scratch)
        assert err(out.cpu().numpy(), O.matmul_f64(xv, dense)) <= TOL, m


def _kats():
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kats.json")
    return json.load(open(path))


def test_reference_kats_through_the_device_decoder(gpu):
    """The reference's own known answers (quant.rs:199-226), decoded on the device: each KAT
    block is row 0, block 0 of a zero 64 x K matrix."""
    kats = _kats()
    for name, type_id, block, bsize in (("q8_0", jq.Q8_0, 32, 34), ("q5_0", jq.Q5_0, 32, 22)):
        n, k = 64, 64
        raw = np.zeros(n * k // block * bsize, np.uint8)
        raw[:bsize] = np.frombuffer(bytes.fromhex(kats[name]["block_hex"]), np.uint8)
        w = jq.QMatrix.upload(gpu, type_id, n, k, 1, raw)
        got = jq.dequant_rows(gpu, w, 0, 1).cpu().numpy()[0]
        for i, v in kats[name]["expect"].items():
            assert got[int(i)] == v, (name, i, got[int(i)])
    # Q4_K: d = dmin = 1, every nibble 1, the KAT's scale bytes: element 32j decodes to s_j - m_j
    kat = kats["q4k_scale_min"]
    n, k = 64, 256
    raw = np.zeros(n * 144, np.uint8)
    raw[0:2] = np.frombuffer(np.array([1.0], np.float16).tobytes(), np.uint8)
    raw[2:4] = raw[0:2]
    raw[4:16] = kat["scale_bytes"]
    raw[16:144] = 0x11
    w = jq.QMatrix.upload(gpu, jq.Q4K, n, k, 1, raw)
    got = jq.dequant_rows(gpu, w, 0, 1).cpu().numpy()[0]
    for j, (sc, mn) in kat["pairs"].items():
        for e in (0, 31):
            assert got[32 * int(j) + e] == float(sc - mn), (j, e, got[32 * int(j) + e])


def test_decode_of_reference_recipes_is_bit_exact(gpu):
    # Q8_0 weights of gpu/tests.rs:431-436 and the Q6_K table of :546-554
    rng = O.Rng(11)
    for type_id, raw, n, k in [(jq.Q8_0, rng.recipe_q8_0(256 * 512 // 32), 256, 512),
                               (jq.Q6K, rng.recipe_q6k(64 * 512 // 256), 64, 512)]:
        w = jq.QMatrix.upload(gpu, type_id, n, k, 1, raw)
        want = O.dequantize(type_id, raw).reshape(n, k)
        got = jq.dequant_rows(gpu, w, 0, n).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), type_id


def test_from_packed_equals_upload(gpu):
    for type_id in (jq.Q4K, jq.Q6K, jq.Q8_0, jq.Q5_0):
        n, k = 64, 512
        raw = synth.weights(type_id, 5, n, k)
        q, h, s, d = O.pack(type_id, raw)
        w = jq.QMatrix.from_packed(gpu, type_id, n, k, 1, q, h, s, d)
        got = jq.dequant_rows(gpu, w, 0, n).cpu().numpy()
        assert np.array_equal(got, O.dequantize(type_id, raw).reshape(n, k)), type_id


# ------------------------------------------------------------------ every plan, small shapes

def all_plans(w, m):
    plans = [jq.Plan(0, 64, 1)]
    for bm in jq.Plan.ROW_TILES:
        for bn in jq.Plan.GFX950_COL_TILES:
            for splits in (1, 2, 8):
                plans.append(jq.Plan(bm, bn, splits))
    plans.append(jq.Plan(256, 128, 1))  # gfx950 Q4_K tile
    return [p for p in plans if p.valid_for(w, m)]


@pytest.mark.parametrize("name,type_id", FORMATS)
@pytest.mark.parametrize("act", ["bf16", "f16", "f32"])
def test_every_plan_matches_oracle_and_tiles_are_row_invariant(gpu, name, type_id, act):
    n, k = 256, 512
    w, raw = make_matrix(gpu, type_id, n, k, seed=7)
    scratch = jq.SplitScratch(gpu)
    gemv_rows = {}
    x_all = synth.normal_rows(100, 150, k)
    for m in (1, 3, 16, 70, 150):
        x32 = x_all[:m]
        x, xv = activations(act, x32)
        if act == "f32":
            xv = xv.astype(np.float16).astype(np.float32)  # the kernels stage FP16 activations
        want = oracle_product(type_id, raw, n, k, xv)
        reference = None
        for plan in all_plans(w, m):
            say(name, act, "m", m, plan)
            out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
            jq.matmul_plan(gpu, x, m, w, out, scratch, plan)
            got = out.cpu().numpy()
            e = err(got, want)
            assert e <= TOL, f"m={m} {plan}: normalized error {e:.2e}"
            if plan.bm == 0:
                gemv_rows[m] = got
            elif plan.splits == 1:
                if reference is None:
                    reference = got
                else:
                    assert np.array_equal(reference, got), f"m={m} {plan} is not row invariant"
    # the small-row kernel computes each row independently of the others
    assert np.array_equal(gemv_rows[1], gemv_rows[3][:1])
    assert np.array_equal(gemv_rows[3], gemv_rows[16][:3])


@pytest.mark.parametrize("name,type_id", FORMATS)
def test_split_k_pipelined_tiles_equal_the_generic_tiles(gpu, name, type_id):
    # Split plans of the pipelined tiles (each slice whole 256-element blocks) against the same
    # splits on the generic kernel (64 x 128): each slice is the same MFMA chain from zero and
    # the partials are summed in the same order, so the bits agree
    n, k = 512, 3072
    w, raw = make_matrix(gpu, type_id, n, k, seed=11)
    scratch = jq.SplitScratch(gpu)
    for m in (37, 100, 256):
        x, xv = activations("bf16", synth.normal_rows(5, m, k))
        want = oracle_product(type_id, raw, n, k, xv)
        for splits in (2, 3, 4):
            reference = None
            for plan in (jq.Plan(64, 128, splits), jq.Plan(64, 64, splits), jq.Plan(128, 128, splits),
                         jq.Plan(256, 128, splits), jq.Plan(32, 64, splits)):
                if not plan.valid_for(w, m):
                    continue
                say(name, "m", m, plan)
                out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
                jq.matmul_plan(gpu, x, m, w, out, scratch, plan)
                got = out.cpu().numpy()
                e = err(got, want)
                assert e <= TOL, f"m={m} {plan}: normalized error {e:.2e}"
                if reference is None:
                    reference = got
                else:
                    assert np.array_equal(reference, got), f"m={m} {plan} differs from the generic split"


@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0)])
def test_small_row_product_of_wide_matrices(gpu, name, type_id):
    """Matrices with at least 8 tiles of 16 rows per compute unit take the persistent small-row
    kernels (activations staged once per workgroup, a range of tiles each): every output against
    the f64 oracle, every row independent of m, and a row of the wide matrix equal to the same
    weight row in a narrow matrix (per-tile kernels at m = 1, persistent ones at m = 5)."""
    cus = gpu.info.compute_units
    n = 64 * (2 * cus + 1)  # 8 tiles per compute unit and 4 more: not a multiple of the grid
    k = 512
    w, raw = make_matrix(gpu, type_id, n, k, seed=11)
    x_all = synth.normal_rows(60, 16, k)
    rows = {}
    for m in (1, 2, 5, 16):
        x, xv = activations("bf16", x_all[:m])
        say(name, "wide", n, k, "m", m)
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, w, out, jq.SplitScratch(gpu))
        got = out.cpu().numpy()
        e = err(got, oracle_product(type_id, raw, n, k, xv))
        assert e <= TOL, f"m={m}: normalized error {e:.2e}"
        rows[m] = got
    assert np.array_equal(rows[1], rows[2][:1])
    assert np.array_equal(rows[2], rows[5][:2])
    assert np.array_equal(rows[5], rows[16][:5])
    # the first 64 weight rows as a matrix of their own run on the per-tile kernels
    per_row = {jq.Q4K: 144 * k // 256, jq.Q6K: 210 * k // 256, jq.Q8_0: 34 * k // 32}[type_id]
    narrow, _ = make_matrix(gpu, type_id, 64, k, seed=0, raw=raw[:64 * per_row].copy())
    for m in (1, 5):
        x, _ = activations("bf16", x_all[:m])
        out = torch.empty((m, 64), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, narrow, out, jq.SplitScratch(gpu))
        assert np.array_equal(out.cpu().numpy(), rows[m][:, :64]), m


@pytest.mark.parametrize("name,type_id,k", [("q4k", jq.Q4K, 3840), ("q4k", jq.Q4K, 2048),
                                             ("q6k", jq.Q6K, 3840), ("q8_0", jq.Q8_0, 4096)])
def test_split_k_small_row_products_equal_the_per_tile_kernels(gpu, monkeypatch, name, type_id, k):
    """Split-K small-row workgroups (W tiles x one of W K slices, the last slice to arrive adding
    the partials; taken here for every m with JV_QMV_SPLIT=1 and a scratch buffer). Their outputs
    must be bitwise those of the per-tile kernels (jv_matvec, no scratch) for every m, match the
    f64 oracle, and keep every row independent of m. 576 rows: a last tile group that is only
    partly filled."""
    monkeypatch.setenv("JV_QMV_SPLIT", "1")
    n = 576
    w, raw = make_matrix(gpu, type_id, n, k, seed=13)
    scratch = jq.SplitScratch(gpu)
    x_all = synth.normal_rows(61, 16, k)
    rows = {}
    for m in (1, 2, 3, 8, 16):
        x, xv = activations("bf16", x_all[:m])
        say(name, "split", n, k, "m", m)
        split = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, w, split, scratch)
        tile = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matvec(gpu, x, m, w, tile)
        got = split.cpu().numpy()
        assert np.array_equal(got, tile.cpu().numpy()), f"m={m}: split-K differs from per-tile"
        e = err(got, oracle_product(type_id, raw, n, k, xv))
        assert e <= TOL, f"m={m}: normalized error {e:.2e}"
        rows[m] = got
    for m in (1, 2, 3, 8):
        assert np.array_equal(rows[m], rows[16][:m]), m
    # the same scratch again, after a split-K tiled product and a product of another format
    # (a different wave count per tile): the tile counters are left at a multiple of 16
    other, _ = make_matrix(gpu, jq.Q8_0 if type_id != jq.Q8_0 else jq.Q4K, 256, 4096, seed=3)
    xo, _ = activations("bf16", synth.normal_rows(5, 4, 4096))
    jq.matmul(gpu, xo, 4, other, torch.empty((4, 256), dtype=torch.float32, device="cuda"), scratch)
    jq.matmul_plan(gpu, xo, 4, other, torch.empty((4, 256), dtype=torch.float32, device="cuda"),
                   scratch, jq.Plan(32, 64, 4))
    for act in ("bf16", "f16", "f32"):
        x, _ = activations(act, x_all[:8])
        a = torch.empty((8, n), dtype=torch.float32, device="cuda")
        b = torch.empty((8, n), dtype=torch.float32, device="cuda")
        for _ in range(2):
            jq.matmul(gpu, x, 8, w, a, scratch)
        jq.matvec(gpu, x, 8, w, b)
        assert np.array_equal(a.cpu().numpy(), b.cpu().numpy()), act
    x, _ = activations("bf16", x_all[:3])
    a16 = torch.empty((3, n), dtype=torch.bfloat16, device="cuda")
    b16 = torch.empty((3, n), dtype=torch.bfloat16, device="cuda")
    jq.matmul(gpu, x, 3, w, a16, scratch)
    jq.matvec(gpu, x, 3, w, b16)
    assert torch.equal(a16, b16)


@pytest.mark.parametrize("name,type_id,k", [("q6k", jq.Q6K, 15360), ("q4k", jq.Q4K, 15360),
                                             ("q8_0", jq.Q8_0, 16384)])
def test_small_row_products_of_long_rows(gpu, name, type_id, k):
    """K too long for the per-tile kernels' per-wave staging at larger m (the down projection,
    K = 15360): the library takes the split-K workgroups, which stage one K slice per
    workgroup, with the caller's scratch buffer or (jv_matvec) the context's own. Outputs
    against the f64 oracle; rows independent of m across the switch from per-tile (small m)
    to split-K kernels."""
    n = 576
    w, raw = make_matrix(gpu, type_id, n, k, seed=17)
    scratch = jq.SplitScratch(gpu)
    x_all = synth.normal_rows(71, 16, k)
    rows = {}
    for m in (1, 4, 8, 16):
        x, xv = activations("bf16", x_all[:m])
        say(name, "long rows", n, k, "m", m)
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, w, out, scratch)
        got = out.cpu().numpy()
        e = err(got, oracle_product(type_id, raw, n, k, xv))
        assert e <= TOL, f"m={m}: normalized error {e:.2e}"
        rows[m] = got
    for m in (1, 4, 8):
        assert np.array_equal(rows[m], rows[16][:m]), m
    # jv_matvec (no scratch buffer) takes the context's own split-K scratch: the same bits
    for m in (8, 16):
        x, _ = activations("bf16", x_all[:m])
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matvec(gpu, x, m, w, out)
        assert np.array_equal(out.cpu().numpy(), rows[m]), m


@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0)])
def test_register_activation_tiles_equal_the_lds_tiles(gpu, monkeypatch, name, type_id):
    """Q4_K, Q6_K and Q8_0 256 x 128, 128 x 128 and 64 x 64 products run by default on waves
    that keep their activation fragments in registers, writing three stages ahead with a
    barrier every second stage; the tiles that share activations through LDS (JV_GEMM_REG=0)
    must give the same bits, and all match the f64 oracle. K = 1024 is four blocks of 8 stages, so
    the steady state, the block switches and the tail all run."""
    n, k, m = 384, 1024, 300
    w, raw = make_matrix(gpu, type_id, n, k, seed=23)
    x, xv = activations("bf16", synth.normal_rows(29, m, k))
    want = oracle_product(type_id, raw, n, k, xv)
    outs = []
    for plan in (jq.Plan(256, 128, 1), jq.Plan(128, 128, 1), jq.Plan(64, 64, 1)):
        for flag in ("1", "0"):
            monkeypatch.setenv("JV_GEMM_REG", flag)
            out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
            jq.matmul_plan(gpu, x, m, w, out, None, plan)
            outs.append(out.cpu().numpy())
            assert err(outs[-1], want) <= TOL, (plan, flag)
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0)])
@pytest.mark.parametrize("k", [256, 512])
def test_eight_wave_tile_short_k_and_bf16_output(gpu, monkeypatch, name, type_id, k):
    """The 8-wave 64 x 64 tile (weight decode split by stage parity) at K of one and two blocks
    of 8 stages (the tail alone, one block switch) with a ragged last row tile: the bits of the
    4-wave tile that shares activations through LDS and of the 4-wave register tile, the f64
    oracle, and a bf16 output equal to the f32 result rounded."""
    n, m = 192, 70
    w, raw = make_matrix(gpu, type_id, n, k, seed=71)
    x, xv = activations("bf16", synth.normal_rows(72, m, k))
    plan = jq.Plan(64, 64, 1)
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("JV_GEMM_REG", flag)
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul_plan(gpu, x, m, w, out, None, plan)
        outs[flag] = out
    assert torch.equal(outs["1"], outs["0"])
    # the 4-wave register tile (the library's choice from two workgroups per CU) alike
    monkeypatch.setenv("JV_GEMM_REG", "1")
    monkeypatch.setenv("JV_GEMM_W8", "0")
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    jq.matmul_plan(gpu, x, m, w, out, None, plan)
    assert torch.equal(outs["1"], out)
    monkeypatch.delenv("JV_GEMM_W8")
    assert err(outs["1"].cpu().numpy(), oracle_product(type_id, raw, n, k, xv)) <= TOL
    monkeypatch.setenv("JV_GEMM_REG", "1")
    o16 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    jq.matmul_plan(gpu, x, m, w, o16, None, plan)
    assert torch.equal(outs["1"].to(torch.bfloat16), o16)


def test_wide_matrix_rows_do_not_depend_on_m_when_the_persistent_kernel_does_not_fit(gpu):
    """A wide Q6_K matrix (8 tiles of 16 rows per compute unit) at K = 3840: the persistent
    small-row kernel's LDS fits up to m = 8 but not at m = 16, where the library takes the
    split-K workgroups (with a scratch buffer) or the per-tile kernels (jv_matvec). Every row
    must have the same bits for every m and kernel, and match the f64 oracle (first 256 rows)."""
    cus = gpu.info.compute_units
    n, k = 16 * 8 * cus, 3840
    raw = synth.weights(jq.Q6K, 31, n, k)
    w = jq.QMatrix.upload(gpu, jq.Q6K, n, k, 1, raw)
    x_all = synth.normal_rows(37, 16, k)
    scratch = jq.SplitScratch(gpu)
    rows = {}
    for m in (1, 8, 16):
        x, xv = activations("bf16", x_all[:m])
        say("q6k wide", n, k, "m", m)
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, w, out, scratch)
        rows[m] = out.cpu().numpy()
        head = raw[:256 * 210 * k // 256].copy()
        e = err(rows[m][:, :256], oracle_product(jq.Q6K, head, 256, k, xv))
        assert e <= TOL, f"m={m}: normalized error {e:.2e}"
    tile = torch.full((16, n), float("nan"), dtype=torch.float32, device="cuda")
    jq.matvec(gpu, activations("bf16", x_all[:16])[0], 16, w, tile)
    assert np.array_equal(tile.cpu().numpy(), rows[16])
    assert np.array_equal(rows[1], rows[16][:1])
    assert np.array_equal(rows[8], rows[16][:8])


@pytest.mark.parametrize("name,type_id,k", [("q4k", jq.Q4K, 3840), ("q6k", jq.Q6K, 3840), ("q8_0", jq.Q8_0, 4096)])
def test_persistent_and_per_tile_kernels_agree_above_two_rows(gpu, monkeypatch, name, type_id, k):
    """Above 2 rows the library streams every matrix with the persistent small-row kernels;
    the per-tile kernels (JV_QMV_PERSIST=0) must give the same bits at every m, and both match
    the f64 oracle."""
    n = 576
    w, raw = make_matrix(gpu, type_id, n, k, seed=41)
    x_all = synth.normal_rows(43, 8, k)
    for m in (3, 4, 5, 8):
        x, xv = activations("bf16", x_all[:m])
        outs = []
        for flag in ("1", "0"):
            monkeypatch.setenv("JV_QMV_PERSIST", flag)
            out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
            jq.matvec(gpu, x, m, w, out)
            outs.append(out.cpu().numpy())
        assert np.array_equal(outs[0], outs[1]), m
        e = err(outs[0], oracle_product(type_id, raw, n, k, xv))
        assert e <= TOL, f"m={m}: normalized error {e:.2e}"


def test_reference_dense_plan_recipe(gpu):
    """every_tunable_dense_plan_matches_reference_and_tiles_are_row_invariant
    (gpu/tests.rs:427-480): Q8_0 N=256 K=512, FP16 rows, every reference plan."""
    n, k = 256, 512
    rng = O.Rng(11)
    raw = rng.recipe_q8_0(n * k // 32)
    w = jq.QMatrix.upload(gpu, jq.Q8_0, n, k, 1, raw)
    dense = O.dequantize(jq.Q8_0, raw).reshape(n, k)
    scratch = jq.SplitScratch(gpu)
    for m in (3, 16, 70, 150):
        xh = rng.h16_vec(m * k, 1.0).reshape(m, k)
        x = torch.from_numpy(xh.astype(np.float16)).cuda()
        want = O.matmul_f64(xh, dense)
        plans = [jq.Plan(0, 128, 1)] + [jq.Plan(bm, bn, s) for bm in jq.Plan.ROW_TILES
                                        for bn in jq.Plan.COL_TILES for s in (1, 2, 8)]
        reference = None
        for plan in [p for p in plans if p.valid_for(w, m)]:
            out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
            jq.matmul_plan(gpu, x, m, w, out, scratch, plan)
            got = out.cpu().numpy()
            assert err(got, want) <= 2e-3 and err(got, want) <= TOL, (m, plan)
            if plan.bm > 0 and plan.splits == 1:
                if reference is None:
                    reference = got
                else:
                    assert np.array_equal(reference, got), (m, plan)


@pytest.mark.parametrize("name,type_id", FORMATS)
def test_tiled_products_use_the_reference_f16_tile(gpu, name, type_id):
    """Identity activations make every output one product 1 * w, so the tiled kernels' outputs
    are their on-chip weight tile: it must equal the reference's f16 tile (the f32 decode of
    quant.rs rounded to nearest even, gemm.rs:131-284) bit for bit."""
    n, k = 128, 512
    say("identity tile", name, n, k)
    w, raw = make_matrix(gpu, type_id, n, k, seed=17)
    tile = O.dequantize(type_id, raw).reshape(n, k).astype(np.float16).astype(np.float32)
    x = torch.eye(k, dtype=torch.float16, device="cuda")
    plans = [jq.Plan(32, 64, 1), jq.Plan(32, 128, 1), jq.Plan(64, 64, 1), jq.Plan(64, 128, 1),
             jq.Plan(128, 64, 1), jq.Plan(128, 128, 1), jq.Plan(256, 128, 1)]
    for plan in [pl for pl in plans if pl.valid_for(w, k)]:
        out = torch.empty((k, n), dtype=torch.float32, device="cuda")
        jq.matmul_plan(gpu, x, k, w, out, None, plan)
        got = out.cpu().numpy()
        want = tile.T.copy() + np.float32(0.0)  # a product's sum of one w and zeros turns -0 into +0
        bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
        detail = [(int(i), int(j), float(got[i, j]), float(want[i, j])) for i, j in bad[:6]]
        assert bad.size == 0, f"{name} {plan}: {len(bad)} elements differ, e.g. (k, n, got, tile) {detail}"


def test_bf16_output_rounds_the_f32_result(gpu):
    n, k, m = 256, 512, 20
    w, raw = make_matrix(gpu, jq.Q4K, n, k, seed=9)
    x, _ = activations("bf16", synth.normal_rows(1, m, k))
    o32 = torch.empty((m, n), dtype=torch.float32, device="cuda")
    o16 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    plan = jq.Plan(32, 128, 1)
    jq.matmul_plan(gpu, x, m, w, o32, None, plan)
    jq.matmul_plan(gpu, x, m, w, o16, None, plan)
    assert torch.equal(o32.to(torch.bfloat16), o16)


# ------------------------------------------------------------------ workload shapes

@pytest.mark.parametrize("m", [1, 4, 8])
def test_q4k_decode_gemv_full_shape(gpu, m):
    """Q4_K GEMV at K=3840, N=15360 (every output checked against the f64 oracle)."""
    n, k = 15360, 3840
    say("q4k gemv", m, n, k)
    w, raw = make_matrix(gpu, jq.Q4K, n, k, seed=2)
    x32 = synth.normal_rows(20 + m, m, k)
    x, xv = activations("bf16", x32)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, out)
    got = out.cpu().numpy()
    want = oracle_product(jq.Q4K, raw, n, k, xv)
    e = err(got, want)
    say("normalized error", e)
    assert e <= TOL
    # split-K workgroups (with a scratch buffer): the same bits
    split = torch.empty((m, n), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, split, jq.SplitScratch(gpu))
    assert np.array_equal(split.cpu().numpy(), got)


def test_q4k_prefill_gemm_m512_rows(gpu):
    """Q4_K GEMM M=512, K=3840, N=15360 with 1% outlier columns: 48 sampled rows against the
    f64 oracle, and rows bitwise equal to another row-invariant plan's on a 16-row slice."""
    m, n, k = 512, 15360, 3840
    say("q4k gemm", m, n, k)
    w, raw = make_matrix(gpu, jq.Q4K, n, k, seed=2)
    x32 = synth.normal_rows(31, m, k, outlier_frac=0.01)
    x, xv = activations("bf16", x32)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    plan = jq.Plan.auto(w, m, row_invariant=True)
    jq.matmul_plan(gpu, x, m, w, out, None, plan)
    got = out.cpu().numpy()
    rows = np.random.default_rng(0).choice(m, 48, replace=False)
    want = oracle_product(jq.Q4K, raw, n, k, xv[rows])
    e = err(got[rows], want)
    say("plan", plan, "normalized error", e)
    assert e <= TOL
    for r0 in (0, 200, 496):
        # the 32 x 64 and 32 x 128 register tiles and the generic tiles (32 x 256)
        for small in (jq.Plan(32, 64, 1), jq.Plan(32, 128, 1), jq.Plan(32, 256, 1)):
            o1 = torch.empty((16, n), dtype=torch.float32, device="cuda")
            jq.matmul_plan(gpu, x[r0:r0 + 16].contiguous(), 16, w, o1, None, small)
            assert torch.equal(o1, out[r0:r0 + 16]), (r0, small)


# ------------------------------------------------------------------ expert-grouped products

def _i32(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).cuda()


@pytest.mark.parametrize("experts,bm,a", [(4, 32, 42), (8, 16, 300), (128, 64, 2048), (3, 128, 5),
                                          (1024, 16, 20000), (128, 64, 4096), (7, 32, 0), (1, 64, 513)])
def test_group_routes_match_the_oracle(gpu, experts, bm, a):
    """ops::group on the device equals its C restatement bitwise (ids >= experts included)."""
    rng = np.random.default_rng(a + experts)
    ids = rng.integers(0, experts + 1, a).astype(np.uint32)
    g = jq.group_routes(gpu, _i32(ids), experts, bm)
    sorted_, offsets, jobs = O.group_routes(ids, experts, bm)
    njobs = int(jobs[0])
    assert g.jobs.cpu().numpy().view(np.uint32)[:1 + 2 * njobs].tolist() == jobs[:1 + 2 * njobs].tolist()
    assert g.offsets.cpu().numpy().view(np.uint32).tolist() == offsets.tolist()
    assert g.ids.cpu().numpy().view(np.uint32)[:sorted_.size].tolist() == sorted_.tolist()


def test_group_routes_far_ids_and_rewrites(gpu):
    """Ids far past the expert count (any bit pattern) are not routed, and a second grouping of
    other routes written into the first one's buffers (`into`) equals the oracle's."""
    experts, bm, a = 100, 32, 3000
    rng = np.random.default_rng(11)
    ids = rng.integers(0, experts, a).astype(np.uint32)
    ids[::7] = rng.integers(experts, 2**32, ids[::7].size, dtype=np.uint64).astype(np.uint32)
    g = jq.group_routes(gpu, _i32(ids), experts, bm)
    ids2 = rng.integers(0, experts, a).astype(np.uint32)
    jq.group_routes(gpu, _i32(ids2), experts, bm, into=g)
    for got, want in ((g, O.group_routes(ids2, experts, bm)),):
        sorted_, offsets, jobs = want
        njobs = int(jobs[0])
        assert got.jobs.cpu().numpy().view(np.uint32)[:1 + 2 * njobs].tolist() == jobs[:1 + 2 * njobs].tolist()
        assert got.offsets.cpu().numpy().view(np.uint32).tolist() == offsets.tolist()
        assert got.ids.cpu().numpy().view(np.uint32)[:sorted_.size].tolist() == sorted_.tolist()
    g1 = jq.group_routes(gpu, _i32(ids), experts, bm)
    sorted_, offsets, jobs = O.group_routes(ids, experts, bm)
    assert g1.offsets.cpu().numpy().view(np.uint32).tolist() == offsets.tolist()
    assert g1.ids.cpu().numpy().view(np.uint32)[:sorted_.size].tolist() == sorted_.tolist()


def test_grouped_products_use_each_assignments_expert_weights(gpu):
    """grouped_products_use_each_assignments_expert_weights (gpu/tests.rs:360-425): Q8_0
    weights of 4 experts (n=128, k=256), 21 tokens routed to 2 experts each, every grouped tile
    and split against the f64 product; tiles without split-K bitwise equal."""
    tokens, top_k, experts, n, k = 21, 2, 4, 128, 256
    rng = O.Rng(3)
    raw = rng.recipe_q8_0(experts * n * k // 32)
    w = jq.QMatrix.upload(gpu, jq.Q8_0, n, k, experts, raw)
    dense = O.dequantize(jq.Q8_0, raw).reshape(experts * n, k)
    x32 = rng.h16_vec(tokens * k, 1.0).reshape(tokens, k)
    x = torch.from_numpy(x32.astype(np.float16)).cuda()
    ids = np.array([(a * 7 + a // top_k) % experts for a in range(tokens * top_k)], np.uint32)
    a = ids.size
    want = O.grouped_product_f64(x32, dense, ids, top_k, n)
    reference = None
    scratch = jq.SplitScratch(gpu)
    for bm in (32, 64):  # GroupPlan::ROW_TILES (gpu/tune.rs:104)
        g = jq.group_routes(gpu, _i32(ids), experts, bm, in_div=top_k)
        for bn in (64, 128):
            for splits in (1, 2):
                out = torch.zeros((a, n), dtype=torch.float32, device="cuda")
                jq.matmul_grouped(gpu, x, w, g, out, bm, bn, splits, scratch)
                got = out.cpu().numpy()
                e = err(got, want)
                assert e <= TOL, f"grouped {bm}x{bn}/{splits}: {e:.2e}"
                if splits == 1:
                    if reference is None:
                        reference = got
                    else:
                        assert np.array_equal(reference, got), f"grouped {bm}x{bn}"
    # the small-row grouped product (jobs of 16 rows)
    g16 = jq.group_routes(gpu, _i32(ids), experts, 16, in_div=top_k)
    out = torch.zeros((a, n), dtype=torch.float32, device="cuda")
    jq.matvec_grouped(gpu, x, w, g16, out, 16)
    assert err(out.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q5_0", jq.Q5_0)])
def test_grouped_products_of_other_formats(gpu, name, type_id):
    """Grouped products of 8 experts with uneven (and one empty) expert loads, bf16 rows, bf16
    and f32 outputs."""
    experts, n, k, top_k, tokens = 8, 128, 512, 2, 37
    raw = synth.weights(type_id, 21, experts * n, k)
    w = jq.QMatrix.upload(gpu, type_id, n, k, experts, raw)
    dense = O.dequantize(type_id, raw).reshape(experts * n, k)
    x, xv = activations("bf16", synth.normal_rows(22, tokens, k))
    rng = np.random.default_rng(23)
    ids = rng.choice([0, 1, 1, 2, 3, 3, 3, 5, 6, 7], tokens * top_k).astype(np.uint32)  # expert 4 empty
    want = O.grouped_product_f64(xv, dense, ids, top_k, n)
    g = jq.group_routes(gpu, _i32(ids), experts, 32, in_div=top_k)
    for out_dtype in (torch.float32, torch.bfloat16):
        out = torch.zeros((ids.size, n), dtype=out_dtype, device="cuda")
        jq.matmul_grouped(gpu, x, w, g, out, 32, 128, 1, None)
        e = err(out.float().cpu().numpy(), want)
        assert e <= (TOL if out_dtype == torch.float32 else 8e-3), (out_dtype, e)


@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0)])
def test_small_row_grouped_products(gpu, monkeypatch, name, type_id):
    """matvec_grouped on the small-row kernels in grouped mode (grid y = job; rows gathered from
    ids / in_div, the expert's weight tiles, output rows scattered to ids): jobs of 1, 2, 4 and
    16 rows, uneven expert loads with an empty expert, K of several items per wave, f32 and
    bf16 outputs, against the f64 oracle and the generic grouped tiles (JV_QMVG=0); every job
    size gives each assignment's row the same bits."""
    experts, n, k, top_k, tokens = 8, 192, 3840 if type_id != jq.Q8_0 else 4096, 2, 21
    raw = synth.weights(type_id, 81, experts * n, k)
    w = jq.QMatrix.upload(gpu, type_id, n, k, experts, raw)
    dense = O.dequantize(type_id, raw).reshape(experts * n, k)
    x, xv = activations("bf16", synth.normal_rows(82, tokens, k))
    rng = np.random.default_rng(83)
    ids = rng.choice([0, 1, 1, 2, 3, 3, 3, 5, 6, 7], tokens * top_k).astype(np.uint32)  # expert 4 empty
    want = O.grouped_product_f64(xv, dense, ids, top_k, n)
    first = None
    for mr in (1, 2, 4, 5, 8, 16):
        g = jq.group_routes(gpu, _i32(ids), experts, mr, in_div=top_k)
        outs = {}
        for flag in ("1", "0"):
            monkeypatch.setenv("JV_QMVG", flag)
            out = torch.full((ids.size, n), float("nan"), dtype=torch.float32, device="cuda")
            jq.matvec_grouped(gpu, x, w, g, out, mr)
            outs[flag] = out.cpu().numpy()
            assert err(outs[flag], want) <= TOL, (mr, flag)
        # one-pass jobs of 1-4 and 5-8 rows and 2-row chunks: the same bits for every job size
        if first is None:
            first = outs["1"]
        assert np.array_equal(outs["1"], first), mr
        monkeypatch.setenv("JV_QMVG", "1")
        o16 = torch.zeros((ids.size, n), dtype=torch.bfloat16, device="cuda")
        jq.matvec_grouped(gpu, x, w, g, o16, mr)
        assert err(o16.float().cpu().numpy(), want) <= 8e-3, mr


@pytest.mark.parametrize("name,type_id,k", [("q4k", jq.Q4K, 256), ("q6k", jq.Q6K, 256), ("q8_0", jq.Q8_0, 512),
                                            ("q4k", jq.Q4K, 2816), ("q6k", jq.Q6K, 1536)])
@pytest.mark.parametrize("act", ["f16", "f32"])
def test_small_row_grouped_products_other_inputs(gpu, monkeypatch, name, type_id, k, act):
    """matvec_grouped as the reference calls it for the down projection (model.rs:968): each
    assignment's own input row (in_div = 1), with f16 activations, and with f32 activations
    through the grouped staging; K = 256 leaves 3 of the 4 waves of the Q4_K / Q6_K grouped
    kernels without items. Jobs of 1, 2, 4 and 16 rows against the f64 oracle."""
    experts, n, top_k, tokens = 8, 128, 2, 13
    raw = synth.weights(type_id, 91, experts * n, k)
    w = jq.QMatrix.upload(gpu, type_id, n, k, experts, raw)
    dense = O.dequantize(type_id, raw).reshape(experts * n, k)
    rng = np.random.default_rng(92)
    ids = rng.choice([0, 1, 1, 2, 3, 3, 3, 5, 6, 7], tokens * top_k).astype(np.uint32)  # expert 4 empty
    x, xv = activations(act, synth.normal_rows(93, tokens * top_k, k))
    if act == "f32":
        xv = xv.astype(np.float16).astype(np.float32)  # the kernels stage FP16 activations
    want = O.grouped_product_f64(xv, dense, ids, 1, n)
    monkeypatch.setenv("JV_QMVG", "1")
    for mr in (1, 2, 4, 16):
        g = jq.group_routes(gpu, _i32(ids), experts, mr, in_div=1)
        out = torch.full((ids.size, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matvec_grouped(gpu, x, w, g, out, mr)
        e = err(out.cpu().numpy(), want)
        say(name, act, "k", k, "mr", mr, "normalized error", e)
        assert e <= TOL, (mr, e)


@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0), ("q5_0", jq.Q5_0)])
def test_grouped_products_on_the_pipelined_tiles(gpu, name, type_id):
    """Grouped jobs of 32 (Q4_K, Q6_K, Q8_0), 64 and 128 rows run on the pipelined tiles (rows
    gathered per job into packed fragments, the expert's weight rows, scattered output rows).
    They must give the bits of the generic grouped tiles (32 x 128 jobs) and match the f64
    oracle, with experts of several jobs, a partly filled last job and an empty expert; f32
    and bf16 outputs."""
    experts, n, k, top_k, tokens = 8, 256, 512, 2, 150
    raw = synth.weights(type_id, 51, experts * n, k)
    w = jq.QMatrix.upload(gpu, type_id, n, k, experts, raw)
    dense = O.dequantize(type_id, raw).reshape(experts * n, k)
    x, xv = activations("bf16", synth.normal_rows(52, tokens, k))
    rng = np.random.default_rng(53)
    ids = rng.choice([0, 0, 0, 1, 1, 2, 3, 3, 3, 3, 5, 6, 7], tokens * top_k).astype(np.uint32)  # expert 4 empty
    want = O.grouped_product_f64(xv, dense, ids, top_k, n)
    g32 = jq.group_routes(gpu, _i32(ids), experts, 32, in_div=top_k)
    ref = torch.full((ids.size, n), float("nan"), dtype=torch.float32, device="cuda")
    jq.matmul_grouped(gpu, x, w, g32, ref, 32, 128, 1, None)
    ref = ref.cpu().numpy()
    assert err(ref, want) <= TOL
    for bm, bn in ((32, 64), (64, 64), (128, 128)):
        g = jq.group_routes(gpu, _i32(ids), experts, bm, in_div=top_k)
        out = torch.full((ids.size, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul_grouped(gpu, x, w, g, out, bm, bn, 1, None)
        assert np.array_equal(out.cpu().numpy(), ref), (bm, bn)
        o16 = torch.zeros((ids.size, n), dtype=torch.bfloat16, device="cuda")
        jq.matmul_grouped(gpu, x, w, g, o16, bm, bn, 1, None)
        assert err(o16.float().cpu().numpy(), want) <= 8e-3, (bm, bn)


# ------------------------------------------------------------------ lm_head argmax

def test_argmax_follows_greedy(gpu):
    s = jq.SplitScratch(gpu)
    rows = [
        [1000.0, 1000.0 + float(np.log(np.float32(2.0))), 0.0],  # model.rs:225-233
        [3.0, 3.0, 1.0],
        [float("inf"), 0.0, 0.0],
        [1.0, float("nan"), 2.0],
        [-1.0, -0.5, -0.5],
    ]
    t = torch.tensor(rows, dtype=torch.float32, device="cuda")
    got = jq.argmax_rows(gpu, t, s).cpu().tolist()
    assert got == [1, 0, -1, -1, 1]
    # ties across chunk boundaries: the first maximum wins
    big = torch.zeros((2, 70000), dtype=torch.float32, device="cuda")
    big[0, 9000] = 5.0
    big[0, 60000] = 5.0
    big[1, 69999] = 1.0
    assert jq.argmax_rows(gpu, big, s).cpu().tolist() == [9000, 69999]
    empty = torch.zeros((3, 0), dtype=torch.float32, device="cuda")
    assert jq.argmax_rows(gpu, empty, s).cpu().tolist() == [-1, -1, -1]


def _greedy_or_minus_one(row):
    try:
        return O.greedy(row)[0]
    except O.OracleError:  # non-finite logits (model.rs:212-214)
        return -1


@pytest.mark.parametrize("n", [1, 3, 5, 1023, 1024, 4097, 65536, 262144])
def test_argmax_random_rows_with_ties(gpu, n):
    """Rows drawn from a few integer values (many ties, first maximum wins), some rows holding a
    NaN or an infinity, on 16-byte aligned rows (vector loads when n % 4 == 0) and on rows that
    start one float past an aligned address (scalar loads), against greedy."""
    s = jq.SplitScratch(gpu)
    rng = np.random.default_rng(n)
    rows = 9
    host = rng.integers(-3, 4, size=(rows, n)).astype(np.float32)
    host[1, rng.integers(0, n)] = np.nan
    host[2, rng.integers(0, n)] = np.inf
    host[3, rng.integers(0, n)] = -np.inf
    host[4] = -5.0  # one value everywhere: index 0
    want = [_greedy_or_minus_one(r) for r in host]
    aligned = torch.from_numpy(host).cuda()
    assert jq.argmax_rows(gpu, aligned, s).cpu().tolist() == want
    buf = torch.empty(rows * n + 1, dtype=torch.float32, device="cuda")
    buf[1:] = aligned.reshape(-1)
    shifted = buf[1:].view(rows, n)
    assert jq.argmax_rows(gpu, shifted, s).cpu().tolist() == want


def test_argmax_repeats_and_graph_replays(gpu):
    """The argmax's partials live in the scratch buffer: consecutive calls on new logits, calls
    interleaved with a split-K small-row product on the same scratch (tile counters and
    partials), and replays of a captured graph with eager work between them all give greedy's
    answers."""
    s = jq.SplitScratch(gpu)
    rng = np.random.default_rng(5)
    rows, n = 8, 262144

    def fresh():
        host = rng.integers(-50, 50, size=(rows, n)).astype(np.float32)
        host[3, rng.integers(0, n)] = np.nan
        return host

    w = jq.QMatrix.upload(gpu, jq.Q4K, 256, 15360, 1, synth.weights(jq.Q4K, 6, 256, 15360))
    x, _ = activations("bf16", synth.normal_rows(7, 16, 15360))
    out = torch.empty((16, 256), dtype=torch.float32, device="cuda")
    for i in range(4):
        host = fresh()
        got = jq.argmax_rows(gpu, torch.from_numpy(host).cuda(), s).cpu().tolist()
        assert got == [_greedy_or_minus_one(r) for r in host], i
        jq.matmul(gpu, x, 16, w, out, s)  # split-K small-row kernel (K = 15360, m = 16)
    t = torch.from_numpy(fresh()).cuda()
    jq.argmax_rows(gpu, t, s)  # buffers grow before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            idx = jq.argmax_rows(gpu, t, s)
    torch.cuda.current_stream().wait_stream(st)
    for i in range(3):
        host = fresh()
        t.copy_(torch.from_numpy(host))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert idx.cpu().tolist() == [_greedy_or_minus_one(r) for r in host], i
        jq.matmul(gpu, x, 16, w, out, s)


@pytest.mark.parametrize("m", [1, 8, 32])
def test_q6k_lm_head_logits_and_argmax(gpu, m):
    """Q6_K vocabulary projection K=3840 on 16384 rows of the vocabulary: logits against the f64
    oracle, argmax equal to the oracle's greedy on the oracle logits wherever the oracle's top-2
    gap exceeds the error bound."""
    n, k = 16384, 3840
    w, raw = make_matrix(gpu, jq.Q6K, n, k, seed=4)
    x, xv = activations("bf16", synth.normal_rows(50 + m, m, k))
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, out, jq.SplitScratch(gpu))
    want = oracle_product(jq.Q6K, raw, n, k, xv)
    e = err(out.cpu().numpy(), want)
    assert e <= TOL
    idx = jq.argmax_rows(gpu, out, jq.SplitScratch(gpu)).cpu().numpy()
    bound = 2 * e * np.abs(want).max()
    for r in range(m):
        srt = np.sort(want[r])
        oracle_idx, _ = O.greedy(want[r].astype(np.float32))
        if srt[-1] - srt[-2] > bound:
            assert idx[r] == int(np.argmax(want[r])), r
        assert idx[r] == O.greedy(out[r].cpu().numpy())[0]


# ------------------------------------------------------------------ lm_head consumers

@pytest.mark.parametrize("name,type_id", [("q6k", jq.Q6K), ("q4k", jq.Q4K), ("q8_0", jq.Q8_0)])
def test_pick_logits_match_the_oracle(gpu, name, type_id):
    """pick_logits (gpu/ops.rs:589-634): softcap(x[row] . E[token]) for (row, token) pairs of a
    1024-token table, against the f64 oracle; out-of-range pairs give NaN."""
    tokens, d, rows, cap = 1024, 768, 6, 30.0
    raw = synth.weights(type_id, 31, tokens, d)
    table = jq.QMatrix.upload(gpu, type_id, tokens, d, 1, raw)
    dense = O.dequantize(type_id, raw).reshape(tokens, d)
    x, xv = activations("f16", synth.normal_rows(32, rows, d))
    rng = np.random.default_rng(33)
    pairs = np.stack([rng.integers(0, rows, 300), rng.integers(0, tokens, 300)], axis=1).astype(np.uint32)
    pairs[7] = pairs[3]  # duplicates
    got = jq.pick_logits(gpu, x, table, torch.from_numpy(pairs.view(np.int32)).cuda(), cap).cpu().numpy()
    want = O.pick_logits_f64(xv, dense, pairs, cap)
    assert np.max(np.abs(got - want)) <= TOL * np.max(np.abs(want))
    assert got[7] == got[3]
    bad = np.array([[rows, 0], [0, tokens], [1, 5]], np.uint32)
    got = jq.pick_logits(gpu, x, table, torch.from_numpy(bad.view(np.int32)).cuda(), cap).cpu().numpy()
    assert np.isnan(got[0]) and np.isnan(got[1]) and np.isfinite(got[2])


def test_softcap_logits(gpu):
    """softcap_logits (gpu/ops.rs:1159-1168) in place against the f64 restatement."""
    v = torch.from_numpy(np.random.default_rng(34).standard_normal(100003).astype(np.float32) * 40).cuda()
    want = O.softcap(v.cpu().numpy(), 30.0)
    jq.softcap_logits(gpu, v, 30.0)
    assert np.max(np.abs(v.cpu().numpy() - want)) <= 4e-6 * 30.0
    with pytest.raises(jq.JvError):
        jq.softcap_logits(gpu, v, 0.0)


# ------------------------------------------------------------------ GGUF -> device

def test_gguf_tensors_upload_unchanged(gpu, tmp_path):
    """The loader step (model.rs:302-351): a [k, n] Q4_K tensor and a [k, n, experts] Q8_0 stack
    read from a GGUF file give the same products as the same bytes uploaded directly."""
    from helpers import write_gguf

    n, k, experts = 128, 512, 3
    q4 = synth.weights(jq.Q4K, 51, n, k)
    q8 = synth.weights(jq.Q8_0, 52, experts * n, k)
    path = str(tmp_path / "w.gguf")
    write_gguf(path, {"general.architecture": (8, "gemma4")},
               [("a.weight", [k, n], 12, q4), ("b.weight", [k, n, experts], 8, q8)])
    g = jq.Gguf(path)
    x, _ = activations("bf16", synth.normal_rows(53, 5, k))
    for name, raw, kind, e in (("a.weight", q4, jq.Q4K, 1), ("b.weight", q8, jq.Q8_0, experts)):
        wf = g.upload(gpu, name)
        wd = jq.QMatrix.upload(gpu, kind, n, k, e, raw)
        assert wf.bytes() == wd.bytes()
        a = jq.dequant_rows(gpu, wf, 0, n * e).cpu().numpy()
        b = jq.dequant_rows(gpu, wd, 0, n * e).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        o1 = torch.empty((5, n), dtype=torch.float32, device="cuda")
        o2 = torch.empty((5, n), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, 5, wf, o1)
        jq.matmul(gpu, x, 5, wd, o2)
        assert torch.equal(o1, o2)
        # ungrouped products of an expert stack use expert 0's rows, as the reference's kernels do
        per_row = raw.size // (n * e)
        w0 = jq.QMatrix.upload(gpu, kind, n, k, 1, raw[:n * per_row].copy())
        o3 = torch.empty((5, n), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, 5, w0, o3)
        assert torch.equal(o1, o3)


# ------------------------------------------------------------------ plan tuner

def test_tuner_measures_stores_and_serves_plans(gpu, tmp_path):
    """Tuner::tune / dense / grouped (gpu/tune.rs:196-343): measured plans are valid for their
    bucket, row-invariant ones split no K, the table reloads for this device, and products with
    the tuned plans match the oracle."""
    path = str(tmp_path / "plans.txt")
    t = jq.Tuner.new(gpu, path)
    n, k = 256, 512
    ws = [make_matrix(gpu, jq.Q4K, n, k, seed=s)[0] for s in (40, 41)]
    raw = synth.weights(jq.Q4K, 40, n, k)
    scratch = jq.SplitScratch(gpu)
    x, xv = activations("bf16", synth.normal_rows(42, 64, k))
    out = torch.empty((64, n), dtype=torch.float32, device="cuda")
    for m, ri in ((64, True), (8, False), (4, True)):
        assert t.tune_dense(ws, m, ri, x, out, scratch)
        p = t.dense(ws[0], m, ri)
        assert p.valid_for(ws[0], m)
        if ri:
            assert p.bm > 0 and p.splits == 1
        o = torch.empty((m, n), dtype=torch.float32, device="cuda")
        jq.matmul_plan(gpu, x[:m].contiguous(), m, ws[0], o, scratch, p)
        assert err(o.cpu().numpy(), oracle_product(jq.Q4K, raw, n, k, xv[:m])) <= TOL
    # grouped tiles for 8 experts, 16 tokens x top-2
    experts, top_k, rows = 8, 2, 16
    wg = jq.QMatrix.upload(gpu, jq.Q8_0, n, k, experts, synth.weights(jq.Q8_0, 43, experts * n, k))
    cap = rows * top_k
    max_jobs = cap // 32 + experts
    route = torch.zeros(cap, dtype=torch.int32, device="cuda")
    sorted_ = torch.zeros(cap, dtype=torch.int32, device="cuda")
    offsets = torch.zeros(experts + 1, dtype=torch.int32, device="cuda")
    jobs = torch.zeros(1 + 2 * (cap + experts), dtype=torch.int32, device="cuda")
    xg, _ = activations("f16", synth.normal_rows(44, cap, k))
    og = torch.empty((cap, n), dtype=torch.float32, device="cuda")
    assert t.tune_grouped([wg], rows, top_k, xg, og, route, sorted_, offsets, jobs, scratch)
    bm, bn = t.grouped(wg, rows)
    assert bm in (32, 64) and bn in (64, 128) and max_jobs > 0
    t.save()
    u = jq.Tuner.new(gpu, path)
    assert u.entries() == t.entries() == 4
    for m, ri in ((64, True), (8, False), (4, True)):
        assert u.dense(ws[0], m, ri) == t.dense(ws[0], m, ri)
    assert u.grouped(wg, rows) == (bm, bn)


# ------------------------------------------------------------------ Burn operator

@pytest.mark.parametrize("m,n,k", [(32, 64, 256), (32, 4160, 512), (64, 256, 1024), (512, 384, 512),
                                   (32, 6144, 4096), (128, 4096, 4096), (32, 28672, 4096)])
def test_f16_matmul_matches_f32_matmul(gpu, m, n, k):
    """f16_matmul_matches_burn_matmul_for_canvas_and_prefill_rows
    (crates/jevons-burn/src/kernels.rs:136-185), tolerance 2e-3 * max(scale, 1)."""
    g = torch.Generator().manual_seed(m * 7 + n)
    x = (torch.rand((m, k), generator=g) * 2 - 1).half()
    wt = ((torch.rand((n, k), generator=g) * 2 - 1) * 0.1).half()
    want = (x.float() @ wt.float().T)
    got = jq.f16_matmul(gpu, x.cuda(), wt.cuda()).cpu()
    worst = (want - got).abs().max().item()
    scale = want.abs().max().item()
    assert worst <= 2e-3 * max(scale, 1.0), worst


def test_f16_matmul_outputs_beyond_the_fp16_range(gpu):
    """kernels.rs:187-218: outputs ~ 1.2e5 come out in full."""
    g = torch.Generator().manual_seed(1)
    x = (29 + 2 * torch.rand((128, 4096), generator=g)).half()
    wt = (0.9 + 0.2 * torch.rand((256, 4096), generator=g)).half()
    want = x.float() @ wt.float().T
    got = jq.f16_matmul(gpu, x.cuda(), wt.cuda()).cpu()
    assert (want - got).abs().max().item() <= want[0, 0].abs().item() * 1e-3


# ------------------------------------------------------------------ host-side rejection

def test_bad_shapes_and_lengths_are_rejected(gpu):
    raw = synth.weights(jq.Q4K, 1, 64, 256)
    with pytest.raises(jq.JvError, match=r"Q4K \[1x64, 256\] has the wrong byte count"):
        jq.QMatrix.upload(gpu, jq.Q4K, 64, 256, 1, raw[:-1])
    with pytest.raises(jq.JvError, match="unsupported type"):
        jq.QMatrix.upload(gpu, 2, 64, 256, 1, raw)
    with pytest.raises(jq.JvError, match=r"Q8_0 \[1x32, 256\] has an unsupported shape"):
        jq.QMatrix.upload(gpu, jq.Q8_0, 32, 256, 1, synth.weights(jq.Q8_0, 1, 32, 256))
    with pytest.raises(jq.JvError, match="F32 has no GPU block layout"):
        jq.QMatrix.upload(gpu, jq.F32, 64, 64, 1, np.zeros(64 * 64 * 4, np.uint8))
    w = jq.QMatrix.upload(gpu, jq.Q4K, 64, 256, 1, raw)
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((4, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(jq.JvError, match="too short"):
        jq.matmul_plan(gpu, x, 5, w, out, None, jq.Plan(32, 64, 1))
    with pytest.raises(jq.JvError, match="not valid"):
        jq.matmul_plan(gpu, x, 4, w, out, None, jq.Plan(48, 64, 1))
    with pytest.raises(jq.JvError, match="not valid"):
        jq.matmul_plan(gpu, x, 4, w, out, None, jq.Plan(32, 128, 1))
    with pytest.raises(jq.JvError, match="at most 16 rows"):
        jq.matvec(gpu, torch.zeros((17, 256), dtype=torch.bfloat16, device="cuda"), 17, w,
                  torch.zeros((17, 64), dtype=torch.float32, device="cuda"))
    with pytest.raises(jq.JvError, match="scratch"):
        jq.matmul_plan(gpu, x, 4, w, out, None, jq.Plan(32, 64, 2))
    # m == 0 is a no-op (gemm.rs:1138, :1219)
    jq.matmul_plan(gpu, x, 0, w, out, None, jq.Plan(32, 64, 1))


def test_plan_rules_follow_the_reference(gpu):
    w = jq.QMatrix.upload(gpu, jq.Q8_0, 256, 512, 1, synth.weights(jq.Q8_0, 1, 256, 512))
    # Plan::heuristic (gemm.rs:987-1004)
    assert jq.Plan.heuristic(w, 70, True, 160) == jq.Plan(64, 128, 1)
    assert jq.Plan.heuristic(w, 2, False, 160) == jq.Plan(0, 128, 1)
    assert jq.Plan.heuristic(w, 16, False, 160) == jq.Plan(32, 128, 2)
    # valid_for (gemm.rs:1006-1015)
    assert jq.Plan(0, 128, 1).valid_for(w, 16) and not jq.Plan(0, 128, 1).valid_for(w, 17)
    assert not jq.Plan(0, 128, 2).valid_for(w, 4)
    assert jq.Plan(128, 128, 8).valid_for(w, 4) and not jq.Plan(128, 128, 9).valid_for(w, 4)
    assert not jq.Plan(128, 128, 0).valid_for(w, 4)
    # the library's own plan: small-row kernel only when rows may differ from the tiles' bits
    assert jq.Plan.auto(w, 4, row_invariant=False).bm == 0
    # row-invariant products of up to 32 rows take the 32 x 64 tile, up to 64 the 64 x 64 one
    assert jq.Plan.auto(w, 4, row_invariant=True) == jq.Plan(32, 64, 1)
    assert jq.Plan.auto(w, 32, row_invariant=True) == jq.Plan(32, 64, 1)
    assert jq.Plan.auto(w, 40, row_invariant=True) == jq.Plan(64, 64, 1)
    # pipelined tiles by rows on a wide matrix (30720 columns, 240 tile columns of 128): 256 x 128
    # from 192 rows, 128 x 128 above 64 rows, 64 x 64 below, while the workgroups fill the device
    if gpu.info.compute_units == 256:
        wide = jq.QMatrix.upload(gpu, jq.Q4K, 30720, 256, 1, synth.weights(jq.Q4K, 1, 30720, 256))
        assert jq.Plan.auto(wide, 256, row_invariant=True) == jq.Plan(256, 128, 1)
        assert jq.Plan.auto(wide, 128, row_invariant=True) == jq.Plan(128, 128, 1)
        assert jq.Plan.auto(wide, 64, row_invariant=True) == jq.Plan(64, 64, 1)
    for m in (1, 4, 16, 70):
        p = jq.Plan.auto(w, m, row_invariant=True)
        assert p.bm > 0 and p.splits == 1 and p.valid_for(w, m), (m, p)
    # the gfx950 256 x 128 tile: any format, whole K in 256-element blocks, split-K only in whole
    # blocks (the generic kernel's slices, z U / splits units)
    assert jq.Plan(256, 128, 1).valid_for(w, 512)
    w320 = jq.QMatrix.upload(gpu, jq.Q8_0, 256, 320, 1, synth.weights(jq.Q8_0, 1, 256, 320))
    assert not jq.Plan(256, 128, 1).valid_for(w320, 512)
    w4 = jq.QMatrix.upload(gpu, jq.Q4K, 256, 512, 1, synth.weights(jq.Q4K, 1, 256, 512))
    assert jq.Plan(256, 128, 1).valid_for(w4, 512) and jq.Plan(256, 128, 2).valid_for(w4, 512)
    assert not jq.Plan(256, 128, 4).valid_for(w4, 512) and not jq.Plan(256, 64, 1).valid_for(w4, 512)
    w8 = jq.QMatrix.upload(gpu, jq.Q8_0, 256, 3840, 1, synth.weights(jq.Q8_0, 1, 256, 3840))
    assert jq.Plan(256, 128, 3).valid_for(w8, 512)  # slices of 20 units (1280 k)
    assert not jq.Plan(256, 128, 8).valid_for(w8, 512)  # 60 units: a slice boundary at 448 k


# ------------------------------------------------------------------ activations beyond FP16

def _wide_range_rows(seed, m, k, act):
    """Rows of BF16 (or F32) values the FP16 staging cannot hold: a plain N(0,1) row; N(0,1)
    x 1e-6 with a few +-1e6 spikes; N(0,1) with one value just above the FP16 maximum; N(0,1)
    x 1e5 everywhere; (F32) 1e30 spikes on N(0,1). Rows repeat cyclically."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    kinds = 5 if act == "f32" else 4
    for r in range(m):
        kind = r % kinds
        if kind == 1:
            x[r] *= np.float32(1e-6)
            cols = rng.choice(k, 5, replace=False)
            x[r, cols] = rng.choice([-1e6, 1e6], 5).astype(np.float32)
        elif kind == 2:
            x[r, rng.integers(0, k)] = np.float32(70000.0)
        elif kind == 3:
            x[r] *= np.float32(1e5)
        elif kind == 4:
            x[r, rng.choice(k, 3, replace=False)] = np.float32(1e30)
    return x


def _row_errors(got, want):
    got = np.asarray(got, np.float64)
    return [float(np.max(np.abs(g - w)) / max(1e-300, np.max(np.abs(w)))) for g, w in zip(got, want)]


@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("name,type_id", [("q4k", jq.Q4K), ("q6k", jq.Q6K), ("q8_0", jq.Q8_0)])
def test_activations_beyond_the_fp16_range(gpu, monkeypatch, name, type_id, act):
    """Rows whose values overflow FP16 (+-1e6 spikes over 1e-6 values, 7e4, 1e5-scale rows, 1e30 in
    F32) through the small-row kernels (per-tile, persistent, split-K), the tiled plans
    (pipelined and generic, with split-K) and the grouped products (pipelined and generic tiles,
    small-row jobs of 1, 2 and 4 rows): every row within 1e-3 of its own largest f64 oracle
    value. A row's power-of-two range scale is exact, so plain rows keep their bits: the small-row
    products of the plain rows alone equal those rows of the mixed batch."""
    n, k = 256, 2048
    raw = synth.weights(type_id, 90, n, k)
    w = jq.QMatrix.upload(gpu, type_id, n, k, 1, raw)
    dense = O.dequantize(type_id, raw).reshape(n, k)
    scratch = jq.SplitScratch(gpu)

    def check(got, want, what):
        errs = _row_errors(got, want)
        assert max(errs) <= TOL, (what, np.argmax(errs), max(errs))

    # small-row kernels
    for m, env in ((1, {}), (4, {}), (4, {"JV_QMV_PERSIST": "0"}), (12, {}), (12, {"JV_QMV_SPLIT": "0"})):
        for kk, v in env.items():
            monkeypatch.setenv(kk, v)
        x32 = _wide_range_rows(91 + m, m, k, act)
        x, xv = activations(act, x32)
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, w, out, scratch)
        got = out.cpu().numpy()
        check(got, O.matmul_f64(xv, dense), ("small-row", m, env))
        plain = [r for r in range(m) if r % (5 if act == "f32" else 4) == 0]
        if len(plain) > 1:  # the plain rows alone: the same bits
            xp, _ = activations(act, x32[plain])
            op = torch.empty((len(plain), n), dtype=torch.float32, device="cuda")
            jq.matmul(gpu, xp, len(plain), w, op, scratch)
            assert np.array_equal(op.cpu().numpy(), got[plain]), ("row invariance", m, env)
        for kk in env:
            monkeypatch.delenv(kk)
    # tiled plans
    m = 40
    x, xv = activations(act, _wide_range_rows(95, m, k, act))
    want = O.matmul_f64(xv, dense)
    tiled = {}
    for plan in (jq.Plan(32, 64, 1), jq.Plan(64, 64, 1), jq.Plan(128, 128, 1), jq.Plan(256, 128, 1),
                 jq.Plan(32, 128, 1), jq.Plan(64, 64, 4)):
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul_plan(gpu, x, m, w, out, scratch, plan)
        tiled[repr(plan)] = out.cpu().numpy()
        check(tiled[repr(plan)], want, plan)
    whole_k = [v for key, v in tiled.items() if "splits: 1" in key]
    for v in whole_k[1:]:  # whole-K plans scale each row alike: the same bits
        assert np.array_equal(v, whole_k[0])
    # grouped products: 4 experts, 30 tokens x top-2
    experts, tokens, top_k = 4, 30, 2
    rawg = synth.weights(type_id, 96, experts * n, k)
    wg = jq.QMatrix.upload(gpu, type_id, n, k, experts, rawg)
    denseg = O.dequantize(type_id, rawg).reshape(experts * n, k)
    x, xv = activations(act, _wide_range_rows(97, tokens, k, act))
    ids = np.random.default_rng(98).integers(0, experts, tokens * top_k).astype(np.uint32)
    want = O.grouped_product_f64(xv, denseg, ids, top_k, n)
    for bm, bn in ((64, 64), (16, 64)):
        g = jq.group_routes(gpu, _i32(ids), experts, bm, in_div=top_k)
        out = torch.full((ids.size, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul_grouped(gpu, x, wg, g, out, bm, bn, 1, None)
        check(out.cpu().numpy(), want, ("grouped", bm, bn))
    for mr in (1, 2, 4):
        g = jq.group_routes(gpu, _i32(ids), experts, mr, in_div=top_k)
        out = torch.full((ids.size, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matvec_grouped(gpu, x, wg, g, out, mr)
        check(out.cpu().numpy(), want, ("grouped small-row", mr))


"""GPU: the vocabulary projection with its soft cap and greedy's argmax in one call
(jv_matmul_argmax; crates/jevons-gemma4-diffusion/src/model.rs:1192-1204, then greedy per row,
crates/jevons-core/src/model.rs:207-219).

Bars: the logits and indices equal, bit for bit, those of jv_matmul, jv_softcap_logits and
jv_argmax_rows in turn, on every kernel family the call takes (persistent small-row kernels and
32 x 64 tiles with the fused epilogue, the other plans through the three steps); every index is
greedy's (the oracle's restatement of model.rs:207-219) on the same logits: first maximum on
ties, -1 for a row holding a non-finite value.
"""
import numpy as np
import pytest
import torch

import jevons_qmm as jq
import oracle as O
from helpers import activations, say
from jevons_qmm import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    yield jq.Gpu(0)


def _greedy_or_invalid(row):
    try:
        return O.greedy(row)[0]
    except O.OracleError:
        return -1


def _three_steps(gpu, x, m, w, n, cap, scratch):
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, out, scratch)
    if cap > 0:
        jq.softcap_logits(gpu, out, cap)
    return out, jq.argmax_rows(gpu, out, scratch)


def _fused(gpu, x, m, w, n, cap, scratch):
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    idx = jq.matmul_argmax(gpu, x, m, w, out, cap, scratch)
    return out, idx


KINDS = [jq.Q4K, jq.Q6K, jq.Q8_0]


@pytest.mark.parametrize("kind", KINDS, ids=["q4k", "q6k", "q8_0"])
@pytest.mark.parametrize("m", [1, 3, 8, 20, 32, 48, 128, 200])
@pytest.mark.parametrize("cap", [0.0, 30.0])
def test_matmul_argmax_equals_the_three_steps(gpu, kind, m, cap):
    """N = 32768 (wide enough for the persistent kernels at M <= 2), K = 512: persistent
    small-row kernels up to M = 16, then the 32 x 64, 64 x 64 (8-wave), 128 x 128 and 256 x 128
    register tiles (M = 200: 56 rows of padding). The weight row j*
    that holds row 0's largest logit is copied into every row j* mod 2048 + 2048 t (other
    workgroups, the same lane and tile position, so the copies' logits are equal bit for bit),
    so greedy must take the first copy, j* mod 2048; row 1 is all zeros (every logit ties:
    index 0) and, from M = 3, row 2 holds a NaN (-1)."""
    n, k = 32768, 512
    raw = synth.weights(kind, 9, n, k).copy()
    x32 = synth.normal_rows(5, m, k)
    if m >= 2:
        x32[1] = 0.0
    if m >= 3:
        x32[2, 5] = np.nan
    x, _ = activations("bf16", x32)
    scratch = jq.SplitScratch(gpu)
    first, _ = _three_steps(gpu, x, m, jq.QMatrix.upload(gpu, kind, n, k, 1, raw), n, 0.0, scratch)
    jstar = O.greedy(first[0].cpu().numpy())[0]
    rows = raw.reshape(n, raw.size // n)
    for t in range(n // 2048):
        rows[jstar % 2048 + 2048 * t] = rows[jstar]
    w = jq.QMatrix.upload(gpu, kind, n, k, 1, raw)
    ref_out, ref_idx = _three_steps(gpu, x, m, w, n, cap, scratch)
    out, idx = _fused(gpu, x, m, w, n, cap, scratch)
    assert torch.equal(out.isnan(), ref_out.isnan())
    assert torch.equal(torch.nan_to_num(out), torch.nan_to_num(ref_out))
    assert torch.equal(idx, ref_idx)
    host, got = out.cpu().numpy(), idx.cpu().numpy()
    for r in range(m):
        assert got[r] == _greedy_or_invalid(host[r]), r
    if cap == 0:  # soft-capped logits may saturate into ties at lower columns
        assert got[0] == jstar % 2048, (jstar, got[0])
    if m >= 2:
        assert got[1] == 0
    if m >= 3:
        assert got[2] == -1
    say("kind", kind, "m", m, "cap", cap, "j*", jstar, "indices", got[:8])


def test_matmul_argmax_on_repeated_calls_and_other_inputs(gpu):
    """Products in a row on one scratch, each smaller and on other weights, the last on the
    per-tile small-row kernel (M = 1 of a narrow matrix), which runs the three steps: each
    call's indices are its own greedy (no stale partials)."""
    scratch = jq.SplitScratch(gpu)
    for seed, m, n, k in ((3, 8, 65536, 1024), (4, 2, 32768, 512), (5, 1, 4096, 512)):
        raw = synth.weights(jq.Q6K, seed, n, k)
        w = jq.QMatrix.upload(gpu, jq.Q6K, n, k, 1, raw)
        x, _ = activations("bf16", synth.normal_rows(seed, m, k))
        out, idx = _fused(gpu, x, m, w, n, 30.0, scratch)
        ref_out, ref_idx = _three_steps(gpu, x, m, w, n, 30.0, scratch)
        assert torch.equal(out, ref_out) and torch.equal(idx, ref_idx)
        host = out.cpu().numpy()
        assert [int(i) for i in idx.cpu()] == [O.greedy(host[r])[0] for r in range(m)]


def test_matmul_argmax_rejects_bad_arguments(gpu):
    n, k = 32768, 256
    w = jq.QMatrix.upload(gpu, jq.Q4K, n, k, 1, synth.weights(jq.Q4K, 1, n, k))
    x, _ = activations("bf16", synth.normal_rows(1, 1, k))
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    scratch = jq.SplitScratch(gpu)
    for cap in (-1.0, float("inf"), float("nan")):
        with pytest.raises(jq.JvError, match="softcap"):
            jq.matmul_argmax(gpu, x, 1, w, out, cap, scratch)


@pytest.mark.parametrize("act,m", [("f32", 3), ("f16", 20), ("bf16", 5), ("bf16", 24)])
def test_matmul_argmax_other_activations_and_range(gpu, act, m):
    """FP32 and FP16 activations, and BF16 rows beyond the FP16 range (divided by a power of
    two before the FP16 rounding and multiplied back, kernels.rs:105, :120-130): the fused call
    equals the three steps bit for bit, on the persistent kernels (M <= 16) and the 32 x 64
    tiles."""
    n, k = 32768, 512
    raw = synth.weights(jq.Q6K, 12, n, k)
    w = jq.QMatrix.upload(gpu, jq.Q6K, n, k, 1, raw)
    x32 = synth.normal_rows(13, m, k)
    if act == "bf16":
        x32[1] *= np.float32(3e5)  # beyond 65504: this row takes a range factor
    x, _ = activations(act, x32)
    scratch = jq.SplitScratch(gpu)
    for cap in (0.0, 30.0):
        ref_out, ref_idx = _three_steps(gpu, x, m, w, n, cap, scratch)
        out, idx = _fused(gpu, x, m, w, n, cap, scratch)
        assert torch.equal(out, ref_out), cap
        assert torch.equal(idx, ref_idx), cap
        host = out.cpu().numpy()
        assert [int(i) for i in idx.cpu()] == [_greedy_or_invalid(host[r]) for r in range(m)]


@pytest.mark.parametrize("cap", [30.0, 1.0, 0.125])
def test_softcap_tanh_accuracy(gpu, cap):
    """The soft cap's tanh (a fitted series below |y| = 0.625, 1 - 2 / (e^(2|y|) + 1) above)
    within 6 ulp of cap tanh(v / cap) computed in f64, over a dense sweep of v / cap in
    [-12, 12] (both branches, the switch point, saturation), tiny and zero values, and +-inf;
    NaN stays NaN."""
    rng = np.random.default_rng(5)
    y = np.concatenate([np.linspace(-12, 12, 2000001), np.linspace(-0.7, 0.7, 400001),
                        np.array([0.625, -0.625, np.nextafter(0.625, 0), 1e-30, -1e-30, 0.0, -0.0, 60.0, -60.0]),
                        rng.standard_normal(100000) * 3]).astype(np.float32)
    v = (y.astype(np.float64) * cap).astype(np.float32)
    t = torch.from_numpy(v.copy()).cuda()
    jq.softcap_logits(gpu, t, cap)
    got = t.cpu().numpy().astype(np.float64)
    want = cap * np.tanh(v.astype(np.float64) / cap)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    err = np.abs(got - want) / np.maximum(ulp, np.spacing(np.float32(0)))
    say("cap", cap, "max ulp", float(err.max()))
    assert err.max() <= 6.0
    special = torch.tensor([np.inf, -np.inf, np.nan], dtype=torch.float32, device="cuda")
    jq.softcap_logits(gpu, special, cap)
    s = special.cpu().numpy()
    assert s[0] == np.float32(cap) and s[1] == -np.float32(cap) and np.isnan(s[2])


@pytest.mark.parametrize("kind,m", [(jq.Q5_0, 20), (jq.Q5_0, 1), (jq.Q4K, 0)])
def test_matmul_argmax_without_epilogue_kernels(gpu, kind, m):
    """Formats without the epilogue variants (Q5_0 runs the generic kernels) take the three
    steps with the same results; M = 0 does nothing."""
    n, k = 4096, 512
    raw = synth.weights(kind, 14, n, k)
    w = jq.QMatrix.upload(gpu, kind, n, k, 1, raw)
    if m == 0:
        x = torch.zeros((1, k), dtype=torch.bfloat16, device="cuda")
        out = torch.zeros((1, n), dtype=torch.float32, device="cuda")
        assert jq.matmul_argmax(gpu, x, 0, w, out, 30.0, jq.SplitScratch(gpu)).numel() == 0
        return
    x, _ = activations("bf16", synth.normal_rows(15, m, k))
    scratch = jq.SplitScratch(gpu)
    for cap in (0.0, 30.0):
        ref_out, ref_idx = _three_steps(gpu, x, m, w, n, cap, scratch)
        out, idx = _fused(gpu, x, m, w, n, cap, scratch)
        assert torch.equal(out, ref_out) and torch.equal(idx, ref_idx), cap


def test_softcap_on_unaligned_and_ragged_buffers(gpu):
    """The soft cap runs four values per thread, with 16-byte accesses where the buffer allows:
    a buffer starting 4 bytes past that alignment, and lengths that are not a multiple of four,
    give the same values as an aligned buffer, and nothing outside the buffer changes."""
    v = np.random.default_rng(17).standard_normal(4099).astype(np.float32) * np.float32(50)
    a = torch.from_numpy(v.copy()).cuda()
    jq.softcap_logits(gpu, a, 30.0)
    b = torch.from_numpy(np.concatenate([np.float32([123.0]), v, np.float32([456.0])])).cuda()
    jq.softcap_logits(gpu, b[1:-1], 30.0)
    assert torch.equal(a, b[1:-1])
    assert float(b[0]) == 123.0 and float(b[-1]) == 456.0
    for n in (1, 2, 3, 5, 7, 1026):
        c = torch.from_numpy(np.concatenate([v[:n], np.float32([789.0])])).cuda()
        jq.softcap_logits(gpu, c[:n], 30.0)
        assert torch.equal(c[:n], a[:n]), n
        assert float(c[n]) == 789.0, n

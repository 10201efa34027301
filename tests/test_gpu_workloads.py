"""GPU parity on the exact workloads bench.py times, against the f64 oracle (quant.rs decode,
f64 matmul):

- one transformer block's six products at M = 256 at their real shapes (Q4_K q, k, v, o,
  gate_up; Q6_K down, K = 15360), and the fused q/k/v projection (N = 4096 + 2 * 2048) the
  reference runs as three launches on one input
  (crates/jevons-gemma4-diffusion/src/model.rs:808-812), on the prefill (whole-K, row
  invariant) plans and on the canvas plans that may split K;
- the Q6_K vocabulary projection over the whole vocabulary (K = 3840, N = 262144) at M = 1, 8
  (persistent small-row kernels) and 32 (32 x 64 tiles), with the per-row argmax of the raw and
  of the soft-capped logits (greedy, crates/jevons-core/src/model.rs:207-219; softcap,
  crates/jevons-gemma4-diffusion/src/gpu/ops.rs:750-758), and the same through the fused call
  (jv_matmul_argmax) bit for bit;
- the Q8_0 GEMV at K = N = 4096 with f32 activations.

Bars: outputs within 1e-3 of max|f64 oracle|; whole-K plans bitwise identical to each other;
argmax equal to greedy on the same logits everywhere, and to the oracle's argmax wherever the
oracle's top-2 gap exceeds the error bound.
"""
import numpy as np
import pytest
import torch

import jevons_qmm as jq
import oracle as O
from helpers import activations, err, oracle_product, say
from jevons_qmm import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
LAYER_M = 256
# name, format, n, k (hidden 3840, 16 heads x 256 for q, 8 x 256 for k and v, FFN 15360)
LAYER = [("q", jq.Q4K, 4096, 3840), ("k", jq.Q4K, 2048, 3840), ("v", jq.Q4K, 2048, 3840),
         ("o", jq.Q4K, 3840, 4096), ("gate_up", jq.Q4K, 30720, 3840), ("down", jq.Q6K, 3840, 15360)]
ROW_INVARIANT_PLANS = [jq.Plan(32, 64, 1), jq.Plan(64, 64, 1), jq.Plan(128, 128, 1), jq.Plan(256, 128, 1),
                       jq.Plan(32, 128, 1)]


@pytest.fixture(scope="module")
def gpu():
    yield jq.Gpu(0)


def _layer_inputs(k, m=LAYER_M):
    return activations("bf16", synth.normal_rows(2, m, k))


def _product(gpu, x, m, w, n, plan):
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    jq.matmul_plan(gpu, x, m, w, out, None, plan)
    return out


@pytest.mark.parametrize("name,kind,n,k", LAYER, ids=[l[0] for l in LAYER])
def test_layer_product_m256_at_its_shape(gpu, name, kind, n, k):
    """The library's prefill plan (row invariant) at the product's real shape: 32 sampled rows
    against the f64 oracle, and every other whole-K plan bitwise equal on all 256 rows."""
    m = LAYER_M
    raw = synth.weights(kind, 5, n, k)
    w = jq.QMatrix.upload(gpu, kind, n, k, 1, raw)
    x, xv = _layer_inputs(k)
    plan = jq.Plan.auto(w, m, row_invariant=True)
    out = _product(gpu, x, m, w, n, plan)
    got = out.cpu().numpy()
    rows = np.sort(np.random.default_rng(11).choice(m, 32, replace=False))
    e = err(got[rows], oracle_product(kind, raw, n, k, xv[rows]))
    say(name, n, k, "plan", plan, "normalized error", e)
    assert e <= TOL
    for other in ROW_INVARIANT_PLANS:
        if other == plan or not other.valid_for(w, m):
            continue
        assert torch.equal(_product(gpu, x, m, w, n, other), out), (name, other)


CANVAS = LAYER + [("qkv", jq.Q4K, 8192, 3840)]


@pytest.mark.parametrize("name,kind,n,k", CANVAS, ids=[l[0] for l in CANVAS])
def test_layer_product_m256_canvas_plans(gpu, name, kind, n, k):
    """The denoising block's canvas plans (row invariance not asked for, split-K allowed:
    Tuner::dense(w, m, false), tune.rs:162-174) at the product's real shape: the library's
    auto plan and the split pipelined tiles the tuner measures, 32 sampled rows each against the
    f64 oracle; a split pipelined plan equals the generic kernel's split of the same slices."""
    m = LAYER_M
    raw = synth.weights(kind, 5, n, k)
    w = jq.QMatrix.upload(gpu, kind, n, k, 1, raw)
    x, xv = _layer_inputs(k)
    rows = np.sort(np.random.default_rng(13).choice(m, 32, replace=False))
    want = oracle_product(kind, raw, n, k, xv[rows])
    scratch = jq.SplitScratch(gpu)
    auto = jq.Plan.auto(w, m, row_invariant=False)
    plans = [auto] + [p for p in (jq.Plan(64, 64, 2), jq.Plan(128, 128, 4), jq.Plan(256, 128, 8)) if p != auto]
    for plan in plans:
        if not plan.valid_for(w, m):
            continue
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        jq.matmul_plan(gpu, x, m, w, out, scratch, plan)
        e = err(out.cpu().numpy()[rows], want)
        say(name, n, k, "canvas plan", plan, "auto" if plan == auto else "", "normalized error", e)
        assert e <= TOL, (name, plan)
        if plan.splits > 1 and plan.bm == 64:
            generic = torch.empty_like(out)
            jq.matmul_plan(gpu, x, m, w, generic, scratch, jq.Plan(64, 128, plan.splits))
            assert torch.equal(generic, out), (name, plan)


def test_fused_qkv_projection_equals_the_three_products(gpu):
    """q, k and v stacked into one Q4_K matrix [8192, 3840]: its product at M = 256 holds the
    three separate products' columns bit for bit, and matches the f64 oracle."""
    m, k = LAYER_M, 3840
    parts = [("q", 4096, 21), ("k", 2048, 22), ("v", 2048, 23)]
    raws = [synth.weights(jq.Q4K, seed, n, k) for _, n, seed in parts]
    fused_raw = np.concatenate(raws)  # GGUF rows are contiguous runs of blocks
    n = sum(p[1] for p in parts)
    wf = jq.QMatrix.upload(gpu, jq.Q4K, n, k, 1, fused_raw)
    x, xv = _layer_inputs(k)
    plan = jq.Plan.auto(wf, m, row_invariant=True)
    fused = _product(gpu, x, m, wf, n, plan)
    c0 = 0
    for (name, nn, _), raw in zip(parts, raws):
        w = jq.QMatrix.upload(gpu, jq.Q4K, nn, k, 1, raw)
        sep = _product(gpu, x, m, w, nn, jq.Plan.auto(w, m, row_invariant=True))
        assert torch.equal(fused[:, c0:c0 + nn], sep), name
        c0 += nn
    rows = np.sort(np.random.default_rng(12).choice(m, 32, replace=False))
    e = err(fused.cpu().numpy()[rows], oracle_product(jq.Q4K, fused_raw, n, k, xv[rows]))
    say("fused qkv plan", plan, "normalized error", e)
    assert e <= TOL


@pytest.fixture(scope="module")
def vocab(gpu):
    """The vocabulary projection's Q6_K table [262144, 3840] (826 MB) and its f32 decode."""
    n, k = 262144, 3840
    raw = synth.weights(jq.Q6K, 4, n, k)
    w = jq.QMatrix.upload(gpu, jq.Q6K, n, k, 1, raw)
    dense = O.dequantize(jq.Q6K, raw).reshape(n, k)
    del raw
    yield n, k, w, dense


def _argmax_checks(gpu, logits, want, bound, what):
    """Device argmax equals greedy on the same logits (every row), and the argmax of the f64
    values `want` wherever their top-2 gap exceeds `bound`; returns the rows inside the bound."""
    idx = jq.argmax_rows(gpu, logits, jq.SplitScratch(gpu)).cpu().numpy()
    host = logits.cpu().numpy()
    close = 0
    for r in range(host.shape[0]):
        assert idx[r] == O.greedy(host[r])[0], (what, r)
        if r in want:
            top2 = np.partition(want[r], -2)[-2:]
            if top2[1] - top2[0] > bound:
                assert idx[r] == int(np.argmax(want[r])), (what, r)
            else:
                close += 1
    return close


@pytest.mark.parametrize("m", [1, 8, 32])
def test_q6k_lm_head_full_vocabulary(gpu, vocab, m):
    """All 262144 logits of every row at M = 1 and 8 (8 sampled rows at M = 32) against the f64
    oracle; argmax of the logits and of the soft-capped logits (cap 30, where saturation makes
    near-ties) as greedy takes it."""
    n, k, w, dense = vocab
    x, xv = activations("bf16", synth.normal_rows(3, m, k))
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, out, jq.SplitScratch(gpu))
    got = out.cpu().numpy()
    rows = np.arange(m) if m <= 8 else np.sort(np.random.default_rng(13).choice(m, 8, replace=False))
    want = O.matmul_f64(xv[rows], dense)
    e = err(got[rows], want)
    say("lm_head m", m, "normalized error", e)
    assert e <= TOL
    wmap = {int(r): want[i] for i, r in enumerate(rows)}
    bound = 2 * float(np.max(np.abs(got[rows] - want)))
    close = _argmax_checks(gpu, out, wmap, bound, "logits")
    cap = 30.0
    _fused_equals(gpu, x, m, w, n, out, 0.0)
    jq.softcap_logits(gpu, out, cap)
    smap = {r: O.softcap(v, cap) for r, v in wmap.items()}
    # tanh is 1-Lipschitz after scaling, and the device tanh adds at most a few ulp of cap
    close_sc = _argmax_checks(gpu, out, smap, bound + 8e-6 * cap, "softcapped")
    _fused_equals(gpu, x, m, w, n, out, cap)
    say("rows within the error bound of a tie:", close, "raw,", close_sc, "soft-capped, of", len(rows))


def _fused_equals(gpu, x, m, w, n, logits, cap):
    """jv_matmul_argmax (product, soft cap and argmax fused) gives `logits` (already soft-capped
    when cap > 0) and their argmax_rows indices bit for bit."""
    scratch = jq.SplitScratch(gpu)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    idx = jq.matmul_argmax(gpu, x, m, w, out, cap, scratch)
    assert torch.equal(out, logits), cap
    assert torch.equal(idx, jq.argmax_rows(gpu, logits, scratch)), cap


@pytest.mark.parametrize("m", [1, 4])
def test_q8_0_gemv_f32_activations_full_shape(gpu, m):
    """Q8_0 GEMV K = N = 4096 with f32 activations (the reference's CPU path input), every output
    against the f64 oracle on the exact f32 values."""
    n = k = 4096
    raw = synth.weights(jq.Q8_0, 3, n, k)
    w = jq.QMatrix.upload(gpu, jq.Q8_0, n, k, 1, raw)
    x, xv = activations("f32", synth.normal_rows(1, m, k))
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, out)
    e = err(out.cpu().numpy(), oracle_product(jq.Q8_0, raw, n, k, xv))
    say("q8_0 f32 m", m, "normalized error", e)
    assert e <= TOL

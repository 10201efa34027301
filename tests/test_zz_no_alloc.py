"""The allocation-free product (jv_matmul_noalloc) against jv_matmul with an allocated scratch
buffer: the same bits on every kernel family that stages through the fixed device array (packed
activations of the tiled products, split-K partials of the generic tiles, split-K small-row
partials and tile counters), on consecutive calls whose inputs shrink, and a clear rejection of a
product whose staging exceeds the array."""
import numpy as np
import pytest
import torch

import jevons_qmm as jq
from helpers import activations, say
from jevons_qmm import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    yield jq.Gpu(0)


def _upload(gpu, kind, n, k, seed):
    return jq.QMatrix.upload(gpu, kind, n, k, 1, synth.weights(kind, seed, n, k))


def _compare(gpu, w, kind, n, k, m, seed):
    x, _ = activations("bf16", synth.normal_rows(seed, m, k))
    want = torch.empty((m, n), dtype=torch.float32, device="cuda")
    got = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, m, w, want, jq.SplitScratch(gpu))
    jq.matmul_noalloc(gpu, x, m, w, got)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (kind, n, k, m)


def test_noalloc_equals_matmul_on_shrinking_inputs(gpu):
    q4 = _upload(gpu, jq.Q4K, 2048, 3840, 1)
    q6 = _upload(gpu, jq.Q6K, 1024, 15360, 2)
    # (matrix, m): the 64 x 64 / 256 x 128 pipelined tiles (packed activations in the array),
    # generic tiles with split-K (partials), persistent and per-tile small-row kernels (no
    # staging), and the split-K small-row kernel of a long K (partials and tile counters)
    calls = [(q4, jq.Q4K, 2048, 3840, 256), (q4, jq.Q4K, 2048, 3840, 64), (q4, jq.Q4K, 2048, 3840, 40),
             (q6, jq.Q6K, 1024, 15360, 8), (q6, jq.Q6K, 1024, 15360, 4), (q4, jq.Q4K, 2048, 3840, 3),
             (q4, jq.Q4K, 2048, 3840, 1)]
    for i, (w, kind, n, k, m) in enumerate(calls):
        say("noalloc", kind, n, k, m)
        _compare(gpu, w, kind, n, k, m, 100 + i)
    # the same product twice in a row, the second smaller, after a larger product of another matrix
    for m in (200, 17):
        say("noalloc again", m)
        _compare(gpu, q4, jq.Q4K, 2048, 3840, m, 300 + m)


def test_noalloc_rejects_staging_beyond_the_array(gpu):
    n, k, m = 2048, 3840, 8192  # packed activations: 8192 x 3840 x 2 B = 60 MiB > 32 MiB
    w = _upload(gpu, jq.Q4K, n, k, 3)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    with pytest.raises(jq.JvError) as e:
        jq.matmul_noalloc(gpu, x, m, w, out)
    import re

    msg = str(e.value)
    assert "fixed scratch array" in msg
    # the message names the staging the product needs (at least its packed activations) and the
    # array's payload
    assert int(re.search(r"needs (\d+) bytes", msg).group(1)) >= m * k * 2
    assert str(jq.NOALLOC_SCRATCH_BYTES - 256 * 1024) in msg
    # nothing ran: the output is untouched, and the entry point still works afterwards
    torch.cuda.synchronize()
    assert not out.any()
    _compare(gpu, w, jq.Q4K, n, k, 64, 7)


def test_noalloc_split_plan_beyond_the_array_runs_whole_k(gpu):
    # the down projection's canvas plan at M = 256 splits K = 15360 eight ways (31.5 MB of
    # partials beside 7.9 MB of packed activations): beyond the array, so the product runs the
    # same 256 x 128 tile with whole K, whose staging fits
    n, k, m = 3840, 15360, 256
    w = _upload(gpu, jq.Q6K, n, k, 4)
    plan = jq.Plan.auto(w, m, row_invariant=False)
    say("noalloc fallback", plan)
    assert plan.splits > 1 and plan.splits * m * n * 4 + m * k * 2 > jq.NOALLOC_SCRATCH_BYTES
    x, xv = activations("bf16", synth.normal_rows(9, m, k))
    got = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    jq.matmul_noalloc(gpu, x, m, w, got)
    whole = torch.empty_like(got)
    jq.matmul_plan(gpu, x, m, w, whole, None, jq.Plan(plan.bm, plan.bn, 1))
    split = torch.empty_like(got)
    jq.matmul(gpu, x, m, w, split, None)  # no scratch given: the context's own holds the partials
    torch.cuda.synchronize()
    assert torch.equal(got, whole)
    ref = torch.empty_like(got)
    jq.matmul_plan(gpu, x, m, w, ref, jq.SplitScratch(gpu), plan)
    assert torch.equal(split, ref)
    scale = whole.abs().max().item()
    assert (split - whole).abs().max().item() <= 1e-4 * scale


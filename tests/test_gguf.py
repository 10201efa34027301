"""GGUF reader (crates/jevons-formats/src/gguf.rs:163-372) through the C ABI, on files written
by tests/helpers.write_gguf; no GPU."""
import numpy as np
import pytest

import jevons_qmm as jq
from helpers import write_gguf
from jevons_qmm import synth


def _model(tmp_path, **kw):
    q4 = synth.weights(jq.Q4K, 1, 64, 512)
    q8 = synth.weights(jq.Q8_0, 2, 4 * 64, 256)  # 4 experts of 64 x 256
    f32 = np.arange(10, dtype=np.float32).tobytes()
    meta = {"general.architecture": (8, "gemma4"), "gemma4.block_count": (4, 30),
            "gemma4.final_logit_softcapping": (6, 30.0), "general.tags": (9, (8, ["a", "bc"])),
            "gemma4.flag": (7, 1), "gemma4.i64": (11, 7)}
    path = str(tmp_path / "m.gguf")
    write_gguf(path, meta, [("blk.0.attn_q.weight", [512, 64], 12, q4),
                            ("blk.0.ffn_down_exps.weight", [256, 64, 4], 8, q8),
                            ("output_norm.weight", [10], 0, f32)], **kw)
    return path, q4, q8, f32


@pytest.mark.parametrize("version,alignment", [(3, None), (2, 64)])
def test_reads_metadata_directory_and_tensor_bytes(tmp_path, version, alignment):
    path, q4, q8, f32 = _model(tmp_path, version=version, alignment=alignment)
    g = jq.Gguf(path)
    assert g.str("general.architecture") == "gemma4"
    assert g.u64("gemma4.block_count") == 30 and g.u64("gemma4.i64") == 7
    assert g.f32("gemma4.final_logit_softcapping") == 30.0
    t = g.tensors()
    assert t["blk.0.attn_q.weight"][:2] == (12, [512, 64]) and t["blk.0.attn_q.weight"][3] == q4.size
    assert t["blk.0.ffn_down_exps.weight"][1] == [256, 64, 4]
    assert all(off % (alignment or 32) == 0 for _, _, off, _ in t.values())
    assert np.array_equal(g.read("blk.0.attn_q.weight"), q4)
    assert np.array_equal(g.read("blk.0.ffn_down_exps.weight", 34 * 8, 34 * 8), q8[34 * 8:34 * 16])  # one expert's rows
    assert g.read("output_norm.weight").tobytes() == f32


def test_errors_carry_the_reference_messages(tmp_path):
    path, *_ = _model(tmp_path)
    g = jq.Gguf(path)
    for call, msg in ((lambda: g.u64("nope"), "Missing GGUF metadata key nope"),
                      (lambda: g.f32("gemma4.block_count"), "is not a float"),
                      (lambda: g.u64("general.architecture"), "is not an unsigned integer"),
                      (lambda: g.read("missing"), "Missing tensor missing"),
                      (lambda: g.read("blk.0.attn_q.weight", 100, 10 ** 9), "range is outside tensor")):
        with pytest.raises(jq.JvError, match=msg):
            call()


@pytest.mark.parametrize("corrupt,msg", [("magic", "bad magic"), ("dup_key", "duplicate metadata key"),
                                         ("misaligned", "is out of bounds"), ("truncate", "is out of bounds")])
def test_rejects_malformed_files(tmp_path, corrupt, msg):
    path, *_ = _model(tmp_path, corrupt=corrupt)
    with pytest.raises(jq.JvError, match="Invalid GGUF file: .*" + msg):
        jq.Gguf(path)


def test_rejects_bad_versions_rows_and_alignment(tmp_path):
    p = str(tmp_path / "v.gguf")
    write_gguf(p, {}, [], version=4)
    with pytest.raises(jq.JvError, match="unsupported version 4"):
        jq.Gguf(p)
    write_gguf(p, {}, [("w", [100, 4], 12, bytes(144 * 2))])
    with pytest.raises(jq.JvError, match="rows are not block aligned"):
        jq.Gguf(p)
    write_gguf(p, {"general.alignment": (4, 24)}, [])
    with pytest.raises(jq.JvError, match="invalid alignment"):
        jq.Gguf(p)

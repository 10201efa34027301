"""Plan tuner rules and table format (crates/jevons-gemma4-diffusion/src/gpu/tune.rs) through the
C ABI, without a GPU."""
import os

import jevons_qmm as jq


def test_row_buckets_cover_each_power_of_two_range():
    """row_buckets_cover_each_power_of_two_range (tune.rs:609-619)."""
    assert jq.tune_bucket(1) == 4
    assert jq.tune_bucket(12) == 16
    assert jq.tune_bucket(16) == 16
    assert jq.tune_bucket(17) == 32
    assert jq.tune_buckets(32, 300) == [32, 64, 128, 256, 512]
    assert jq.tune_buckets(4, 1) == [4]
    assert jq.tune_buckets(4, 12) == [4, 8, 16]
    assert jq.tune_buckets(32, 4096) == [32, 64, 128, 256, 512, 1024]


def test_heuristic_plan_is_kept_unless_clearly_slower():
    """heuristic_plan_is_kept_unless_clearly_slower (tune.rs:601-607): ids 0 = 'h', 1 = 'a',
    2 = 'b'; the baseline is 'h'."""
    assert jq.tune_pick([1.00, 0.97], [0, 1], 0) == 0
    assert jq.tune_pick([1.00, 0.90], [0, 1], 0) == 1
    assert jq.tune_pick([0.80, 0.90], [1, 2], 0) == 0
    assert jq.tune_pick([], [], 0) is None


def test_plan_table_round_trip(tmp_path):
    """Tuner::save / load (tune.rs:358-444): entries written under the profile line come back;
    another profile's table is ignored; malformed lines are skipped."""
    path = str(tmp_path / "plans.txt")
    t = jq.Tuner.open_table("v1 device=0 cus=256 wave=64 lds=163840 arch=gfx950", path)
    assert t.entries() == 0
    t.insert_dense(jq.FMT_Q4K, 4096, 3840, 256, True, jq.Plan(64, 64, 1))
    t.insert_dense(jq.FMT_Q4K, 4096, 3840, 8, False, jq.Plan(32, 128, 4))
    t.insert_grouped(jq.FMT_Q8_0, 128, 256, 4, 32, 64, 128)
    t.save()
    text = open(path).read().splitlines()
    assert text[0] == t.profile
    assert "dense 0 4096 3840 8 0 32 128 4" in text and "dense 0 4096 3840 256 1 64 64 1" in text
    assert "grouped 3 128 256 4 32 64 128" in text
    with open(path, "a") as f:
        f.write("dense 1 2 3\nnonsense line\n")
    u = jq.Tuner.open_table(t.profile, path)
    assert u.entries() == 3
    assert u.lookup_dense(jq.FMT_Q4K, 4096, 3840, 200, True) == jq.Plan(64, 64, 1)  # bucket 256
    assert u.lookup_dense(jq.FMT_Q4K, 4096, 3840, 100, True) is None
    assert u.lookup_dense(jq.FMT_Q4K, 4096, 3840, 5, False) == jq.Plan(32, 128, 4)
    other = jq.Tuner.open_table("v1 device=1 cus=256 wave=64 lds=163840 arch=gfx950", path)
    assert other.entries() == 0
    assert not os.path.exists(path + ".tmp")

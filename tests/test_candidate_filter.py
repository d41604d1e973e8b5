"""Host tests of the tile-manifest filter (behaviour of
src/axon/candidate_filter.py:17-173 in the reference)."""

from axon.candidate_filter import (
    MANIFEST_NAME,
    TileConstraint,
    manifest_literal,
    read_manifest,
    rejection_reason,
    select_diverse,
)


def test_block_must_fit_extent():
    c = TileConstraint("TILES_IN_BLOCK_N", 512, 512, False)
    assert c.rejection_reason(1) is None
    assert "block 1024 > extent 512" in c.rejection_reason(2)
    assert "not positive" in c.rejection_reason(0)


def test_divisibility():
    c = TileConstraint("TILES_IN_BLOCK_N", 768, 128, True)
    assert c.rejection_reason(2) is None
    assert "does not divide extent 768" in c.rejection_reason(4)


def test_manifest_round_trip(tmp_path):
    cons = (
        TileConstraint("TILES_IN_BLOCK_N", 512, 512, False),
        TileConstraint("TILES_IN_BLOCK_M", 128, 128, True),
    )
    mod = tmp_path / "k.py"
    mod.write_text(f"{MANIFEST_NAME} = {manifest_literal(cons)}\n")
    # The literal is written sorted by tile_arg.
    assert read_manifest(mod) == tuple(sorted(cons, key=lambda c: c.tile_arg))


def test_fail_open_cases(tmp_path):
    assert read_manifest(tmp_path / "missing.py") == ()
    dyn = tmp_path / "dyn.py"
    dyn.write_text(f"{MANIFEST_NAME} = build()\n")
    assert read_manifest(dyn) == ()
    fut = tmp_path / "fut.py"
    fut.write_text(f"{MANIFEST_NAME} = {{'version': 2, 'constraints': ()}}\n")
    assert read_manifest(fut) == ()
    dup = tmp_path / "dup.py"
    rec = "{'tile_arg': 'TILES_IN_BLOCK_M', 'extent': 1, 'tile_size': 1, 'require_divisible': False}"
    dup.write_text(f"{MANIFEST_NAME} = ({rec}, {rec})\n")
    assert read_manifest(dup) == ()
    bad = tmp_path / "bad.py"
    bad.write_text("def (:\n")
    assert read_manifest(bad) == ()


def test_unversioned_tuple_is_accepted(tmp_path):
    mod = tmp_path / "old.py"
    mod.write_text(
        f"{MANIFEST_NAME} = ({{'tile_arg': 'TILES_IN_BLOCK_M', 'extent': 64, 'tile_size': 32, "
        "'require_divisible': True},)\n"
    )
    assert read_manifest(mod) == (TileConstraint("TILES_IN_BLOCK_M", 64, 32, True),)


def test_rejection_reason_matches_by_name():
    cons = (TileConstraint("TILES_IN_BLOCK_N", 512, 512, False),)
    args = ("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N")
    assert rejection_reason(args, (32, 1), cons) is None
    assert rejection_reason(args, (1, 2), cons) is not None


def test_select_diverse_bounded_deterministic_with_corners():
    cands = [(m, n) for m in (1, 2, 4, 8) for n in (1, 2, 4, 8)]
    sel = select_diverse(cands, budget=8, seed=42)
    assert len(sel) == 8 and sel == sorted(sel)
    assert sel == select_diverse(list(reversed(cands)), budget=8, seed=42)
    for corner in ((1, 1), (8, 8), (1, 8), (8, 1)):
        assert corner in sel


def test_select_diverse_known_answer():
    """Hand-derived: one axis of {1, 2, 4, 8}, budget 3. Anchors (1,) and
    (8,) come first; then (4,) beats (2,): 0.65*2/3 + 0.35*1/3 = 0.55 against
    0.65*1/3 + 0.35*1/3 = 1/3."""
    assert select_diverse([(1,), (2,), (4,), (8,)], budget=3, seed=42) == [(1,), (4,), (8,)]


def test_zero_budget_and_small_pools_keep_everything():
    assert select_diverse([(4,), (1,), (2,), (2,)], budget=0, seed=1) == [(1,), (2,), (4,)]
    assert select_diverse([(1, 2)], budget=8, seed=1) == [(1, 2)]

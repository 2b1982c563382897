"""CPU: host decisions of the level pipeline (no GPU calls): the query-table load a level's index is sized at."""

import pytest

from ngram_amd import partcount
from ngram_amd.levels import DENSE_LOAD, LevelBuild
from ngram_amd.qindex import EXPECT_MARGIN, LOAD, TAIL


def _engine(contexts: dict, density: dict | None = None, wide=()) -> LevelBuild:
    lb = LevelBuild.__new__(LevelBuild)  # only the learnt sizes _load reads; no tokens, no library
    lb.contexts_of = dict(contexts)
    lb.density = dict(density or {})
    lb.wide = set(wide)
    return lb


def _ids(expect: int, load: float) -> int:
    # the slots QueryIndex gives a table sized from `expect` contexts at `load` (its cap plus the tail)
    return int(expect * EXPECT_MARGIN / load) + 1024 + TAIL


def test_dense_levels_take_the_sparser_table():
    # c3's level-2 context count: both loads give 25-bit ids and the count's runs mode
    lb = _engine({2: 4_276_390, 3: 9_903_899})
    assert lb._load(2, None, 4, None) == DENSE_LOAD
    # level 3 behind a dense level 2 (density >= 0.5: a lane per position) likewise
    lb.density[2] = 0.79
    assert lb._load(3, 2, 4, None) == DENSE_LOAD


def test_default_load_without_a_learnt_count_or_behind_a_sparse_level():
    lb = _engine({3: 9_903_899}, density={2: 0.3})
    assert lb._load(2, None, 4, None) is None  # no count learnt yet (a cold build): sized for every position
    assert lb._load(3, 2, 4, None) is None  # behind a sparser level its scan lists positions: not every one probed


def test_default_load_off_the_32_bit_count():
    lb = _engine({2: 4_276_390}, wide={2})
    assert lb._load(2, None, 4, None) is None  # a level the 64-bit count takes
    assert _engine({2: 4_276_390})._load(2, None, 8, 4) is None  # the TOP rule's build


@pytest.mark.parametrize("ktop", [4, 8])
def test_default_load_where_the_sparser_table_changes_the_count_layout(ktop):
    # a context count whose table fits the runs mode at the default load but not at DENSE_LOAD (its ids one bit
    # wider): the level keeps the default, so the count's layout is what it would be without the rule
    expect = next(e for e in range(1 << 20, 1 << 28, 1 << 16)
                  if partcount.runs_fit(_ids(e, LOAD), ktop) and not partcount.runs_fit(_ids(e, DENSE_LOAD), ktop))
    assert _engine({2: expect})._load(2, None, ktop, None) is None

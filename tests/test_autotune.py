"""Host logic of the split autotuner (testtimeideas_amd/autotune.py): the
candidates around the library's pick, the choice of the fastest, caching per
shape, and the cases that keep the library's own choice."""
import pytest

from testtimeideas_amd import autotune


@pytest.fixture(autouse=True)
def _state(monkeypatch):
    prev = autotune.enabled()
    autotune.clear()
    monkeypatch.setattr(autotune, "_capturing", lambda: False)
    yield
    autotune.enable(prev)
    autotune.clear()


def test_candidates_start_with_the_pick_and_stay_in_range():
    assert autotune.candidates(20, 128) == [20, 10, 15, 25, 30, 40, 128]
    assert autotune.candidates(4, 6) == [4, 5, 6]       # 2 and 3 clip to the smallest split, 8 to the walk
    assert autotune.candidates(3, 3) == [3]             # a walk shorter than the smallest split
    assert autotune.candidates(128, 128) == [128, 64, 96]


def test_off_returns_library_choice_without_timing(monkeypatch):
    autotune.enable(False)
    monkeypatch.setattr(autotune, "_time", lambda run, c: pytest.fail("timed while off"))
    assert autotune.chunk(("k",), lambda: pytest.fail("asked while off"), lambda c: None) == 0


def test_picks_fastest_and_caches(monkeypatch):
    autotune.enable(True)
    cost = {20: 5.0, 10: 7.0, 15: 4.0, 25: 4.5, 30: 6.0, 40: 9.0, 128: 30.0}
    timed = []
    monkeypatch.setattr(autotune, "_time", lambda run, c: (timed.append(c), cost[c])[1])
    assert autotune.chunk(("a",), lambda: (20, 128), lambda c: None) == 15
    assert sorted(timed) == sorted(cost)
    timed.clear()
    assert autotune.chunk(("a",), lambda: pytest.fail("re-tuned"), lambda c: None) == 15
    assert timed == []
    assert autotune.choices() == {("a",): 15}


def test_ties_keep_the_library_pick(monkeypatch):
    autotune.enable(True)
    monkeypatch.setattr(autotune, "_time", lambda run, c: 1.0)
    assert autotune.chunk(("b",), lambda: (20, 128), lambda c: None) == 0  # the library's own pick


def test_single_candidate_is_not_timed(monkeypatch):
    autotune.enable(True)
    monkeypatch.setattr(autotune, "_time", lambda run, c: pytest.fail("timed a single candidate"))
    assert autotune.chunk(("c",), lambda: (3, 3), lambda c: None) == 0


def test_graph_capture_keeps_library_choice(monkeypatch):
    autotune.enable(True)
    monkeypatch.setattr(autotune, "_capturing", lambda: True)
    monkeypatch.setattr(autotune, "_time", lambda run, c: pytest.fail("timed during capture"))
    assert autotune.chunk(("d",), lambda: (20, 128), lambda c: None) == 0
    assert autotune.choices() == {}

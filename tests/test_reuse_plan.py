"""q35m_reuse_plan: the prefix-reuse plan of KvCacheAlign.Plan
(src/Qwen35Sharp.Model/KvCacheAlign.cs:20-28) through the C ABI (host only),
the reference's KvCacheAlignTests (tests/Qwen35Sharp.Tests/
KvCacheAlignTests.cs:7-53) ported fact by fact, a brute-force restatement of
the plan on random id lists, and the snapshot extension: the kept length moves
back to the longest snapshot not past the reference's plan."""
import random

import pytest

import q35mix


def plan(cached, prompt, snaps=()):
    return q35mix.reuse_plan(cached, prompt, snaps)


# --- KvCacheAlignTests, one test per fact ---------------------------------

def test_diverging_tail_keeps_shared_prefix():
    cached, prompt = [1, 2, 3, 4, 5], [1, 2, 3, 6, 7]
    t, s, snap = plan(cached, prompt)
    assert (t, s, snap) == (3, 3, -1)
    assert prompt[s:] == [6, 7]


def test_longer_cache_than_prompt_does_not_drop_prefix():
    cached, prompt = [1, 2, 3, 10, 11], [1, 2, 3, 6]
    t, s, _ = plan(cached, prompt)
    assert t == 3
    assert prompt[s:] == [6]


def test_full_hit_replays_last_token():
    ids = [1, 2, 3]
    t, s, _ = plan(ids, ids)
    assert (t, s) == (2, 2)
    assert ids[s:] == [3]


def test_empty_cache_forwards_whole_prompt():
    prompt = [4, 5, 6]
    t, s, _ = plan([], prompt)
    assert t == 0
    assert prompt[s:] == prompt


def test_no_overlap_resets():
    assert plan([1, 2, 3], [9, 8])[:2] == (0, 0)


# --- the plan restated, on random id lists ----------------------------------

def reference_plan(cached, prompt):
    """KvCacheAlign.Plan as written: CommonPrefixLength, then the full-hit rule."""
    if not prompt:
        return 0
    n, i = min(len(cached), len(prompt)), 0
    while i < n and cached[i] == prompt[i]:
        i += 1
    return len(prompt) - 1 if i == len(prompt) else i


def test_random_lists_match_restatement():
    rng = random.Random(5)
    for _ in range(2000):
        base = [rng.randrange(4) for _ in range(rng.randrange(12))]
        cached = base[:rng.randrange(len(base) + 1)] + [rng.randrange(4) for _ in range(rng.randrange(4))]
        prompt = base[:rng.randrange(len(base) + 1)] + [rng.randrange(4) for _ in range(rng.randrange(4))]
        want = reference_plan(cached, prompt)
        assert plan(cached, prompt) == (want, want, -1), (cached, prompt)


def test_empty_prompt_and_prompt_inside_cache():
    assert plan([1, 2, 3], []) == (0, 0, -1)
    assert plan([], []) == (0, 0, -1)
    # A prompt that is a prefix of the cache is a full hit: all but its last token.
    assert plan([1, 2, 3, 4], [1, 2]) == (1, 1, -1)


# --- snapshot extension -----------------------------------------------------

def test_snapshot_longest_not_past_plan():
    cached, prompt = [1, 2, 3, 4, 5, 6], [1, 2, 3, 4, 9]     # reference plan: keep 4
    assert plan(cached, prompt, [2, 6, 0, 4, 3]) == (4, 4, 3)
    assert plan(cached, prompt, [2, 6, 3]) == (3, 3, 2)
    assert plan(cached, prompt, [5, 6]) == (0, 0, -1)     # none fits: reset
    # Full hit: the last token is replayed, so a snapshot at the prompt's full
    # length does not fit.
    assert plan([1, 2, 3], [1, 2, 3], [3, 1]) == (1, 1, 1)
    assert plan([1, 2, 3], [1, 2, 3], [3]) == (0, 0, -1)


def test_invalid_arguments():
    lib = q35mix.lib()
    import ctypes
    out = [ctypes.c_int(0) for _ in range(3)]
    refs = [ctypes.byref(o) for o in out]
    assert lib.q35m_reuse_plan(None, -1, None, 0, None, 0, *refs) == q35mix.ERR_INVALID
    assert lib.q35m_reuse_plan(None, 2, None, 0, None, 0, *refs) == q35mix.ERR_INVALID
    assert lib.q35m_reuse_plan(None, 0, None, 0, None, 0, None, refs[1], refs[2]) == q35mix.ERR_INVALID
    with pytest.raises(q35mix.Q35Error) as ei:
        q35mix.check(lib.q35m_reuse_plan(None, 0, None, 1, None, 0, *refs))
    assert ei.value.code == q35mix.ERR_INVALID

"""When a linear-state snapshot is still restorable (CPU; no device).

The library's rule (qwen3.5sharp_amd/csrc/snapshot_marks.h, used by
q35m_snapshot_restore / q35m_snapshot_valid) is checked against a brute-force
model of one sequence that records a version number for every K/V row: a
snapshot is restorable exactly when the rows below its length carry the
versions they had at the save (and the sequence is at least that long).  The
model's events are those of the library: decode/prefill appends rows at the
current length, truncate, reset, restore of a snapshot, and K/V state writes
of rows from 0.  Random histories must agree on every query.

A multi-turn prefix reuse (the scenario q35m_reuse_plan serves) shows why the
host passes only accepted snapshots to the plan: after a later turn
restores a shorter snapshot and forwards new tokens, a longer snapshot of the
first turn is refused, and the plan over the accepted lengths picks the
snapshot the restore then accepts.
"""
import os
import random
import subprocess

import pytest

import q35mix

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("marks") / "marks")
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "qwen3.5sharp_amd", "csrc"),
                    os.path.join(ROOT, "tests", "snapshot_marks_driver.cpp"), "-o", exe], check=True)
    return exe


class Marks:
    """The library's DropMarks through the driver process."""

    def __init__(self, exe):
        self.p = subprocess.Popen([exe], stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True, bufsize=1)

    def _ask(self, line):
        self.p.stdin.write(line + "\n")
        self.p.stdin.flush()
        return self.p.stdout.readline().strip()

    def save(self):
        return int(self._ask("save"))

    def drop(self, n):
        self.p.stdin.write(f"drop {n}\n")
        self.p.stdin.flush()

    def valid(self, stamp, kv, cur):
        return self._ask(f"valid {stamp} {kv} {cur}") == "1"

    def entries(self):
        return int(self._ask("entries"))

    def close(self):
        self.p.stdin.close()
        assert self.p.wait() == 0


class Sequence:
    """Brute-force model: per-row versions, the length, and the library's
    marks driven by the same events."""

    def __init__(self, marks, cap=64):
        self.m = marks
        self.rows = [0] * cap
        self.len = 0
        self.version = 0
        self.snaps = []            # (stamp, kv_len, row versions below kv_len)

    def append(self, k):
        for r in range(self.len, self.len + k):
            self.version += 1
            self.rows[r] = self.version
        self.len += k

    def truncate(self, x):
        if x < self.len:
            self.m.drop(x)
        self.len = x

    def reset(self):
        self.m.drop(0)
        self.len = 0

    def kv_write(self, n):
        self.m.drop(0)
        for r in range(n):
            self.version += 1
            self.rows[r] = self.version

    def save(self):
        self.snaps.append((self.m.save(), self.len, list(self.rows[:self.len])))
        return len(self.snaps) - 1

    def truth(self, i):
        _, kv, rows = self.snaps[i]
        return kv <= self.len and self.rows[:kv] == rows

    def lib_valid(self, i):
        stamp, kv, _ = self.snaps[i]
        return self.m.valid(stamp, kv, self.len)

    def restore(self, i):
        _, kv, _ = self.snaps[i]
        if kv < self.len:
            self.m.drop(kv)
        self.len = kv


@pytest.mark.parametrize("seed", range(40))
def test_rule_matches_row_versions(driver, seed):
    rng = random.Random(seed)
    m = Marks(driver)
    s = Sequence(m)
    checked = 0
    for _ in range(300):
        ev = rng.random()
        if ev < 0.35 and s.len < 60:
            s.append(rng.randint(1, min(4, 60 - s.len)))
        elif ev < 0.50:
            s.save()
        elif ev < 0.62 and s.len:
            s.truncate(rng.randint(0, s.len))
        elif ev < 0.65:
            s.reset()
        elif ev < 0.68:
            s.kv_write(rng.randint(1, 8))
        elif s.snaps:
            i = rng.randrange(len(s.snaps))
            truth = s.truth(i)
            assert s.lib_valid(i) == truth, (seed, i, s.snaps[i][:2], s.len)
            checked += 1
            if truth and rng.random() < 0.5:
                s.restore(i)
        # every snapshot agrees after every event
        for i in range(len(s.snaps)):
            assert s.lib_valid(i) == s.truth(i), (seed, i)
    assert checked > 10
    assert m.entries() <= 64
    m.close()


def test_multi_turn_prefix_reuse(driver):
    """Turn 1 forwards prompt P1 (12 tokens) saving snapshots at 3, 6 and 9.
    Turn 2's prompt keeps 7 tokens: the plan picks the snapshot at 6, which
    is restored, and 7 new tokens are forwarded with snapshots at 8 and 12.
    Turn 3's prompt keeps 10 tokens of that history: the snapshot at 9 (of
    turn 1, before the cut to 6) is refused; the plan over the accepted
    lengths picks 8, which the restore accepts."""
    m = Marks(driver)
    s = Sequence(m)
    snap_at = {}
    p1 = list(range(100, 112))
    for i in range(len(p1)):
        s.append(1)
        if s.len in (3, 6, 9):
            snap_at[s.len] = s.save()
    cached = p1
    p2 = p1[:7] + [200 + i for i in range(6)]           # 13 tokens, common prefix 7
    idx = [snap_at[3], snap_at[6], snap_at[9]]
    lens = [s.snaps[i][1] for i in idx]
    ok = [i for i in idx if s.lib_valid(i)]
    assert len(ok) == 3
    trunc, start, pick = q35mix.reuse_plan(cached, p2, [s.snaps[i][1] for i in ok])
    assert (trunc, start) == (6, 6) and lens[pick] == 6
    s.restore(ok[pick])
    for t in range(start, len(p2)):
        s.append(1)
        if s.len in (8, 12):
            snap_at[s.len] = s.save()
    cached = p2
    p3 = p2[:10] + [300, 301]                           # common prefix 10
    candidates = [snap_at[3], snap_at[6], snap_at[9], snap_at[8], snap_at[12]]
    # without filtering the plan would take the snapshot at 9, which restore refuses
    t_all, _, pick_all = q35mix.reuse_plan(cached, p3, [s.snaps[i][1] for i in candidates])
    assert t_all == 9 and not s.lib_valid(candidates[pick_all]) and not s.truth(candidates[pick_all])
    ok = [i for i in candidates if s.lib_valid(i)]
    assert [s.snaps[i][1] for i in ok] == [3, 6, 8, 12]
    trunc, start, pick = q35mix.reuse_plan(cached, p3, [s.snaps[i][1] for i in ok])
    assert (trunc, start) == (8, 8) and s.snaps[ok[pick]][1] == 8
    assert s.lib_valid(ok[pick]) and s.truth(ok[pick])
    s.restore(ok[pick])
    assert s.len == 8
    m.close()

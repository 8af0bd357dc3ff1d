// Host-only: whether the K/V rows below a snapshot's length are unchanged
// since the snapshot was saved.
//
// A linear-state snapshot (q35m_snapshot_save) holds the DeltaNet states of a
// sequence at length Ls; restoring it is sound only while the sequence's K/V
// rows [0, Ls) are the ones the saved states went with.  Mixers write rows at
// or above the current length only, so rows below Ls can change only after
// the length has dropped below Ls: a truncation, a restore to a shorter
// length, a reset (to 0), or a K/V state write (rows from 0, counted as a
// drop to 0).  DropMarks keeps, per sequence, a clock that ticks at every
// save and every drop, and the drops as a stack of (tick, length) with ticks
// and lengths both increasing from the bottom: a new drop to length x first
// removes every entry of length >= x (for any save before those entries the
// new drop is also later and no higher), so the lowest length dropped to
// after tick t is the length of the first entry whose tick exceeds t.  A
// snapshot saved at tick t with length Ls is restorable iff that lowest
// length is >= Ls (and the sequence is at least Ls long).
#pragma once

#include <climits>
#include <cstdint>
#include <utility>
#include <vector>

namespace q35 {

class DropMarks {
public:
    // Stamp of a save.
    uint32_t save() { return ++tick_; }
    // The length dropped to `len` (or rows from 0 were rewritten: len 0).
    void drop(int len) {
        const uint32_t t = ++tick_;
        while (!stack_.empty() && stack_.back().second >= len) stack_.pop_back();
        stack_.emplace_back(t, len);
    }
    // Lowest length dropped to after stamp t (INT_MAX when none).
    int lowest_since(uint32_t t) const {
        size_t lo = 0, hi = stack_.size();
        while (lo < hi) {
            const size_t mid = (lo + hi) / 2;
            if (stack_[mid].first > t) hi = mid;
            else lo = mid + 1;
        }
        return lo < stack_.size() ? stack_[lo].second : INT_MAX;
    }
    // A snapshot of length kv_len stamped t, at current length cur.
    bool restorable(uint32_t t, int kv_len, int cur) const {
        return t != 0 && t <= tick_ && kv_len >= 0 && kv_len <= cur && lowest_since(t) >= kv_len;
    }
    size_t entries() const { return stack_.size(); }

private:
    uint32_t tick_ = 0;
    std::vector<std::pair<uint32_t, int>> stack_;
};

}  // namespace q35

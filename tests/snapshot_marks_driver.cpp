// Test driver for q35::DropMarks (qwen3.5sharp_amd/csrc/snapshot_marks.h),
// built with g++ by tests/test_snapshot_marks.py.  Reads one command per
// line from stdin and prints one line per query:
//   save                 -> prints the stamp
//   drop <len>
//   valid <stamp> <kv_len> <cur>  -> prints 1 or 0
//   entries              -> prints the stack size
#include <cstdio>
#include <cstring>

#include "snapshot_marks.h"

int main() {
    std::setvbuf(stdout, nullptr, _IOLBF, 0);   // one answer per line, read interactively
    q35::DropMarks m;
    char cmd[32];
    while (std::scanf("%31s", cmd) == 1) {
        if (!std::strcmp(cmd, "save")) {
            std::printf("%u\n", m.save());
        } else if (!std::strcmp(cmd, "drop")) {
            int len = 0;
            if (std::scanf("%d", &len) != 1) return 2;
            m.drop(len);
        } else if (!std::strcmp(cmd, "valid")) {
            unsigned t = 0;
            int kv = 0, cur = 0;
            if (std::scanf("%u %d %d", &t, &kv, &cur) != 3) return 2;
            std::printf("%d\n", m.restorable(t, kv, cur) ? 1 : 0);
        } else if (!std::strcmp(cmd, "entries")) {
            std::printf("%zu\n", m.entries());
        } else {
            return 2;
        }
    }
    return 0;
}

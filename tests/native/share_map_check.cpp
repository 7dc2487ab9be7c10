// Host-only check of the fused kernel's work partition (detail::ShareMap in
// iq_gemv.h): for every (grid, heads, splits per head) given on stdin, each
// split of each head lies in exactly one workgroup's share, each workgroup's
// share splits into runs whose split slots are distinct and fill [0, nr) per
// head, and nr <= splits per head (so the slots fit the workspace).
// Input lines: grid heads splits e0_num.  Prints "ok <paired>" or
// "FAIL <reason>" per line.
#include <cstdio>
#include <vector>

#include "../../innerq_amd/csrc/iq_gemv.h"

using iq::detail::ShareMap;

int main() {
  int grid, nhead, nsplit, e0num;
  while (std::scanf("%d %d %d %d", &grid, &nhead, &nsplit, &e0num) == 4) {
    const ShareMap m = ShareMap::make(grid, nhead, nsplit, e0num);
    std::vector<int> cover(size_t(nhead) * nsplit, 0);
    std::vector<std::vector<int>> slots(nhead);
    const char* err = nullptr;
    std::vector<int> seen_share(size_t(2) * grid, 0);
    for (int b = 0; b < grid && !err; ++b) {
      int side = 0, sh = 0;
      m.share(b, side, sh);
      if (sh < 0 || sh >= m.width() || (side && !m.paired)) { err = "share index"; break; }
      if (seen_share[size_t(side) * grid + sh]++) { err = "two workgroups on one share"; break; }
      const int64_t i0 = m.begin(side, sh), i1 = m.begin(side, sh + 1);
      const int L = m.len(side);
      for (int64_t j = i0; j < i1;) {  // runs: maximal pieces of one head
        const int h = int(j / L);
        const int64_t e = i1 < int64_t(h + 1) * L ? i1 : int64_t(h + 1) * L;
        for (int64_t t = j; t < e; ++t) cover[size_t(h) * nsplit + m.first(side) + (t - int64_t(h) * L)]++;
        if (!m.paired && (m.share_of(j) != sh || m.share_of(e - 1) != sh)) { err = "share_of"; break; }
        slots[h].push_back(m.slot(side, sh, h));
        j = e;
      }
    }
    for (size_t i = 0; i < cover.size() && !err; ++i)
      if (cover[i] != 1) err = "split not covered exactly once";
    for (int h = 0; h < nhead && !err; ++h) {
      const int nr = m.nruns(h);
      if (int(slots[h].size()) != nr || nr > nsplit) { err = "run count"; break; }
      std::vector<int> used(nr, 0);
      for (int s : slots[h]) {
        if (s < 0 || s >= nr || used[s]++) { err = "slot"; break; }
      }
    }
    if (err) std::printf("FAIL %s\n", err);
    else std::printf("ok %d\n", m.paired);
  }
  return 0;
}

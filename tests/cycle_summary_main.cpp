// Host check of grxCycleSummarize from include/grx/grx_cycles.h: reads
// "start end core warp" lines from stdin and prints
// "warps cores spanIsValid span busyMin busyMedian busyMax".
#include <grx/grx_cycles.h>

#include <cstdio>
#include <vector>

int main() {
  std::vector<grxCycleSlot> slots;
  unsigned long long start = 0, end = 0;
  unsigned core = 0, warp = 0;
  while (std::scanf("%llu %llu %u %u", &start, &end, &core, &warp) == 4)
    slots.push_back(grxCycleSlot{start, end, core, warp});
  grxCycleSummary s;
  grxCycleSummarize(slots.data(), (int)slots.size(), &s);
  std::printf("%d %d %d %llu %llu %llu %llu\n", s.warps, s.cores, s.spanIsValid,
              (unsigned long long)s.span, (unsigned long long)s.busyMin,
              (unsigned long long)s.busyMedian, (unsigned long long)s.busyMax);
  return 0;
}

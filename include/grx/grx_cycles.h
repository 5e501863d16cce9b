/* grx_cycles.h -- per-wave cycle records written by the library's kernels.
 *
 * Same slot layout as the reference's measurement ABI
 * (ref: include/grx/grx_cycles.h:38-54) so that a benchmark written against it
 * reads the records unchanged. On gfx950 `start`/`end` come from the wave's
 * s_memtime shader clock and `core` identifies the hardware unit that ran the
 * wave (XCD in the high half, CU in the low half): clocks of different XCDs
 * are not comparable, so a span across them is reported as invalid.
 */
#ifndef GRX_CYCLES_H
#define GRX_CYCLES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  uint64_t start;
  uint64_t end;
  uint32_t core;
  uint32_t warp;
} grxCycleSlot;

typedef struct {
  int      warps;
  int      cores;
  int      spanIsValid;
  uint64_t span;
  uint64_t busyMin;
  uint64_t busyMedian;
  uint64_t busyMax;
} grxCycleSummary;

#ifdef __cplusplus
}  /* extern "C" */

#include <algorithm>
#include <vector>

/* Host-only summary of a slot array (semantics of the reference's
 * grxCycleSummarize, ref: include/grx/grx_cycles.h:67-99): all-zero slots were
 * never written and are skipped; the span is only meaningful when every
 * written slot came from one clock domain. */
inline void grxCycleSummarize(const grxCycleSlot* slots, int n,
                              grxCycleSummary* out) {
  if (!out) return;
  *out = grxCycleSummary{};
  if (!slots || n <= 0) return;
  std::vector<uint64_t> busy;
  busy.reserve((size_t)n);
  uint64_t lo = UINT64_MAX, hi = 0;
  uint32_t domain = 0;
  bool single = true, any = false;
  for (int i = 0; i < n; ++i) {
    const grxCycleSlot& s = slots[i];
    if (s.start == 0 && s.end == 0) continue;
    if (!any) { domain = s.core; any = true; }
    else if (s.core != domain) single = false;
    lo = std::min(lo, s.start);
    hi = std::max(hi, s.end);
    busy.push_back(s.end - s.start);
  }
  if (busy.empty()) return;
  std::sort(busy.begin(), busy.end());
  out->warps       = (int)busy.size();
  out->cores       = single ? 1 : 2;
  out->spanIsValid = single ? 1 : 0;
  out->span        = single ? hi - lo : 0;
  out->busyMin     = busy.front();
  out->busyMedian  = busy[busy.size() / 2];
  out->busyMax     = busy.back();
}
#endif  /* __cplusplus */

#endif  /* GRX_CYCLES_H */

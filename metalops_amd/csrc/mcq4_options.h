// Test and experiment switches of the library, read from the environment once
// (at the first launch) and again only on mcq4_reload_options(), never per
// call.  opt(name) returns the value of a known MCQ4_* variable as it was at
// the last (re)load, or nullptr when it was unset.
#pragma once

#include <stdint.h>

namespace mcq4 {
const char *opt(const char *name);
// True when the named switch is set and its value starts with `c`.
inline bool opt_is(const char *name, char c) {
    const char *v = opt(name);
    return v && v[0] == c;
}
// Splits of an XCD-local split-K exchange that the kernels treat as having run
// on another XCD (bit q = split q): MCQ4_SPLIT_FOREIGN, a test switch that
// drives the recompute path on hardware where the placement always holds.
uint32_t split_foreign_mask();
// Polls of a split-K flag before the waiting workgroup recomputes that split
// (MCQ4_SPLIT_SPIN, default 256, at most 2^20; 0 drives the recompute path
// for every other split).
uint32_t split_spin();
}  // namespace mcq4

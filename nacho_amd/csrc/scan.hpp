// Device-wide exclusive prefix sum of int64 counts (scan.hip).
#pragma once

#include <cstdint>

#include "runtime.hpp"

namespace nacho {
namespace scan {

// out[i] = in[0] + ... + in[i-1] for i in [0, n]; out has n + 1 entries (out[n] = total).
// Runs on the call's stream; scratch comes from the call.
int exclusive_scan_i64(Call &call, const int64_t *in, int64_t n, int64_t *out);

}  // namespace scan
}  // namespace nacho

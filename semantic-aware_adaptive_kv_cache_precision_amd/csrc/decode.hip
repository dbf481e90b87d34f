// The decode attention fast path: one query per head, 32-token pages.
//
// Until the matrix-core decode kernel lands, every launch goes to the
// general kernel in attention.hip.

#include "common.hpp"
#include "kernels.hpp"

namespace mi
{
  bool launch_decode_fast(const KVSource &, const AttentionArgs &, hipStream_t) { return false; }
} // namespace mi

// Per-row decode bookkeeping shared by the greedy and the sampled token
// choosers (one thread per row calls it after the row's token is known).
#pragma once

#include "common.hpp"

namespace grpo {

// The reference's per-row bookkeeping of a decode step (paged_kv.py:800-820,
// :938, :978) for the chosen token g of row m: record it, advance the lengths,
// stop at EOS or the row's limit, set the next step's append slot and attention
// length.
__device__ __forceinline__ void advance_row(int m, int64_t g, int64_t* tokens, int32_t* pos,
                                            int32_t* count, const int32_t* limit,
                                            uint8_t* active, const int64_t* eos,
                                            int64_t* generated, int64_t gen_ld,
                                            int32_t* append_pos, int32_t* attn_len) {
  const bool a = active[m] != 0;
  if (a) {
    const int c = count[m];
    if (generated && c >= 0 && c < gen_ld) generated[(int64_t)m * gen_ld + c] = g;
    pos[m] += 1;
    count[m] = c + 1;
  }
  const bool still = a && count[m] < limit[m] && g != eos[0];
  active[m] = still ? 1 : 0;
  tokens[m] = g;
  append_pos[m] = still ? pos[m] : -1;
  attn_len[m] = still ? pos[m] + 1 : 0;
}

}  // namespace grpo

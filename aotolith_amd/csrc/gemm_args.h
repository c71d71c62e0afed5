// Kernel-argument record of the prefill GEMM's RoPE epilogue (w4_gemm.h), shared
// by the device code and the host launcher: one plain struct passed by value.
#pragma once

#include <stdint.h>

namespace aoto {

// The q/k/v projection's RoPE and cache fill at batch 1 (the arguments of
// aoto_rope_qkv_prefill): rotated queries to q_out[h][m][D], rotated keys and
// the values to pair[0|1][h][slot0 + m][D] of a [2][Hkv][cap][D] window, table
// row positions[m]; with zero_prefix, slots [0, slot0) of both are zeroed.
struct QkvRope {
  const long long* positions;
  const uint16_t* cos_table;
  const uint16_t* sin_table;
  uint16_t* q_out;
  uint16_t* pair;
  int query_heads;
  int kv_heads;
  int head_dim;
  int cap;
  int slot0;
  int zero_prefix;
};

}  // namespace aoto

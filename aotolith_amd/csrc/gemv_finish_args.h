// Arguments of the greedy loop's argmax finish when it runs in the prologue of
// the next step's first GEMV (w4_gemv_stream.h, FINISH). Shared by the kernel
// and the host launcher, which passes it by value as the kernel's last
// argument (plain pointers and integers: the same layout on both sides).
#pragma once

#include <stdint.h>

namespace aoto {

// The greedy loop's argmax finish, done in the prologue of the next step's first
// GEMV (FINISH): every block reduces the previous LM head's `count` per-wave
// keys to the token and stages that token's embedding row as x; block 0 also
// records it as aoto_argmax_finish does - token_out, the history entry, the
// step state advanced by one token, the advanced position's RoPE rows, and the
// raw embedding row into hidden_out (the step's residual); a token outside the
// table's `embed_rows` rows stages zeros and sets error[0]. Null pointers skip
// the history, step state, RoPE rows or error flag.
struct GemvFinishArgs {
  long long* token_out;
  long long* history;
  int* history_len;
  int* step;
  const uint16_t* cos_table;
  const uint16_t* sin_table;
  uint16_t* rope_rows;
  uint16_t* hidden_out;
  int* error;
  long long embed_rows;
  int count;  // keys (the finish kernel takes it packed among its first arguments)
  int cap;
  int head_dim;
};

}  // namespace aoto

// Host+device shared internals of libsdv (not part of the public ABI).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "sdv.h"
#include "sdv_device.h"

namespace sdv {

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Where the new tokens of an append go when the caller gives no slot mapping: token b*q_len + i
// is position T_b - q_len + i of sequence b (T_b = seq_lens[b], or max_seq_len for every
// sequence when seq_lens is NULL), placed through the block table.
struct SlotTable {
  const int32_t* block_table;
  int32_t max_blocks;
  const int32_t* seq_lens;
  int32_t q_len;
  int32_t max_seq_len;
};

// sdv_quant_append with the slots taken from a SlotTable (no slot mapping).
int quant_append_table(const void* v_new, const void* k_new, const SlotTable& table, int32_t n_tokens,
                       int32_t kv_heads, int32_t head_dim, int32_t num_layers, int64_t in_layer_stride,
                       void* k_pages, void* v_pages, float* v_scales, int32_t num_blocks, int64_t k_layer_stride,
                       int64_t v_layer_stride, int64_t s_layer_stride, int32_t scale_mode, void* stream);

}  // namespace sdv

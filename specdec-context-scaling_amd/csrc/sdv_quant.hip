// Kernel 1: fused V-only FP8 quantize + paged append (and the BF16 K copy).
//
// Restates, per (token, KV head), specdec/engine/model_self.py:304-314 with group_size ==
// head_dim (the v_fp8 format, model_self.py:690,703): s = max|v| / 448 (s == 0 -> 1),
// payload = RNE_E4M3FN(v / s), and the append of payload, scale and BF16 K
// (model_self.py:721-722, 795-799) -- written into pages instead of concatenated.
//
// K is copied into the page's [D/8][16][8] chunk layout (see include/sdv.h).
//
// One wavefront handles 16 consecutive input tokens of one KV head of one layer (or, with a
// caller's tile table, the up-to-16 rows of one table entry: a batched varlen prefill passes
// tiles that start where each sequence starts, so whole page blocks keep the 16-byte stores
// although sequences start anywhere in the packed input); a workgroup holds four such
// wavefronts.  D/8 lanes (a "row") hold one token's
// head_dim values as 16-byte pieces, so each wave-wide load brings 64/(D/8) whole token rows
// and a lane ends up holding J = 16 / rows consecutive tokens of the same 8 dimensions.  The
// max-abs of a token is a DPP reduction inside its row (no cross-row traffic).  The V page
// is dimension-major ([D][16 tokens] bytes), so when the 16 tokens fill one page block
// exactly (prefill) each lane packs its J codes per dimension, the wave transposes them
// through LDS, and every dimension's 16 codes leave as one 16-byte store; otherwise (decode,
// partial or scattered blocks) codes go out as single bytes per slot.  K moves as 16-byte
// pieces from its loads, issued with the V loads before any arithmetic, to its page chunk.
//
// The kernel is VALU-bound if each value takes an IEEE division and a branchy encoder, so
// per token it forms r = RN(1/s) once, and per value takes RN(x / s) as one multiply and two
// fma (quotient_rn) and converts with v_cvt_pk_fp8_f32 (gfx950: OCP E4M3FN, round to
// nearest even; equal to the integer encoder for every fp32 input except the sign of a NaN,
// which cannot occur on this route).  Tokens whose max-abs is not finite or lies in
// (0, 2^-60) take the exact division and the integer encoder instead.
#include "sdv_internal.h"

namespace sdv {

struct QuantArgs {
  const uint16_t* v_new;
  const uint16_t* k_new;
  const int32_t* slots;
  const int32_t* tiles;  // optional tile table: tile i = rows [tiles[i], min(tiles[i] + 16, tiles[i+1]))
  int n_tiles;
  int n_tokens;
  int kv_heads;
  int num_blocks;
  int scale_mode;
  int64_t in_ls;
  uint16_t* k_pages;
  uint8_t* v_pages;
  float* v_scales;
  int64_t k_ls, v_ls, s_ls;
  SlotTable table;  // used when slots == nullptr
};

// slot of input row `row`: from the caller's mapping, or through the block table
__device__ __forceinline__ int row_slot(const QuantArgs& a, int row) {
  if (a.slots) return a.slots[row];
  const int b = row / a.table.q_len, i = row - b * a.table.q_len;
  const int T = a.table.seq_lens ? min(max(a.table.seq_lens[b], 0), a.table.max_seq_len) : a.table.max_seq_len;
  return table_slot(a.table.block_table + (int64_t)b * a.table.max_blocks, a.table.max_blocks, a.num_blocks,
                    T - a.table.q_len + i);
}

constexpr int kQuantWaves = 4;  // wavefronts (16-token tiles) per workgroup

template <int D, bool WITH_K, bool TABLE>
__global__ __launch_bounds__(64 * kQuantWaves) void quant_append_kernel(QuantArgs a) {
  constexpr int LPR = D / 8;          // lanes per token row: 16 bytes of BF16 each
  constexpr int RPW = kWave / LPR;    // token rows per wave-wide load (4 or 8)
  constexpr int J = kBlock / RPW;     // consecutive tokens held by one lane (4 or 2)
  // per wavefront: the codes of one page block, [D][16 tokens] bytes
  __shared__ uint4 lds_codes[kQuantWaves][D];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane / LPR, p = lane % LPR;
  const int tile = blockIdx.x * kQuantWaves + wave;
  int t0, nt;
  if constexpr (TABLE) {  // rows from the caller's table, clamped to the input
    if (tile >= a.n_tiles) return;  // wave-uniform
    t0 = min(max(a.tiles[tile], 0), a.n_tokens);
    nt = min(min(a.tiles[tile + 1], a.n_tokens) - t0, kBlock);
    if (nt <= 0) return;
  } else {  // 16 consecutive rows
    t0 = tile * kBlock;
    if (t0 >= a.n_tokens) return;  // wave-uniform
    nt = min(kBlock, a.n_tokens - t0);
  }
  const int kvh = blockIdx.y;
  const int layer = blockIdx.z;
  const int KV = a.kv_heads;

  const uint16_t* vin = a.v_new + layer * a.in_ls;
  const uint16_t* kin = a.k_new + layer * a.in_ls;
  uint16_t* kp = a.k_pages + layer * a.k_ls;
  uint8_t* vp = a.v_pages + layer * a.v_ls;
  float* sp = a.v_scales + layer * a.s_ls;

  // slots first (unconditional loads from a clamped index, so that all of them are in flight
  // together), then every V and K load: the arithmetic below waits on the slots only
  // V: lane (r, p) holds tokens r*J .. r*J+J-1; K (no per-token arithmetic) is read with
  // token j*RPW + r in load j, so that the lanes storing one page chunk hold consecutive tokens
  int slot[J], kslot[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    slot[j] = row_slot(a, t0 + min(r * J + j, nt - 1));
    if (WITH_K) kslot[j] = row_slot(a, t0 + min(j * RPW + r, nt - 1));
  }
  // rows past the end of the input re-read the last token (skipped below): no branches
  // around the loads, so that none of them has to land before the slots are used
  uint4 vw[J], kw[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    vw[j] = load_stream16(vin + ((int64_t)(t0 + min(r * J + j, nt - 1)) * KV + kvh) * D + 8 * p);
    if (WITH_K) kw[j] = load_stream16(kin + ((int64_t)(t0 + min(j * RPW + r, nt - 1)) * KV + kvh) * D + 8 * p);
  }

  const int64_t n_slots = (int64_t)a.num_blocks * kBlock;
#pragma unroll
  for (int j = 0; j < J; ++j) {  // past the end or out of range: skipped
    if (r * J + j >= nt || (int64_t)slot[j] >= n_slots) slot[j] = -1;
    if (WITH_K && (j * RPW + r >= nt || (int64_t)kslot[j] >= n_slots)) kslot[j] = -1;
  }
  const int slot0 = __builtin_amdgcn_readlane(slot[0], 0);
  bool contiguous = true;
#pragma unroll
  for (int j = 0; j < J; ++j) contiguous = contiguous && slot[j] == slot0 + r * J + j;
  const bool full = nt == kBlock && slot0 >= 0 && (slot0 & (kBlock - 1)) == 0 && __ballot(!contiguous) == 0;

  // per token: scale s, its correctly rounded reciprocal, and whether the fast route holds
  float scale[J], rcp[J];
  bool fast[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t mb = abs_max_bits8(vw[j]);
    token_scale(row_max_bits<LPR>(mb), a.scale_mode, scale[j], rcp[j], fast[j]);
  }

  // codes: packed[k] holds dimension k's J codes, token j in byte j
  uint32_t packed[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float q[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t wk = (k & 1) ? (&vw[j].x)[k >> 1] & 0xFFFF0000u : (&vw[j].x)[k >> 1] << 16;
      q[j] = quotient_rn(__uint_as_float(wk), scale[j], rcp[j]);
    }
    uint32_t c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    if (J == 4) c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2 % J], q[3 % J], (int)c, true);
    packed[k] = c;
  }
  // tokens outside the fast route (max-abs non-finite, or in (0, 2^-60)): exact division and
  // the integer encoder, byte by byte (rare; skipped when no lane of the wave has one)
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (fast[j]) continue;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t wk = (k & 1) ? (&vw[j].x)[k >> 1] & 0xFFFF0000u : (&vw[j].x)[k >> 1] << 16;
      const uint32_t code = e4m3fn_encode(__uint_as_float(wk) / scale[j]);
      packed[k] = (packed[k] & ~(0xFFu << (8 * j))) | (code << (8 * j));
    }
  }

  if (!full) {  // decode, partial or scattered blocks: one byte per slot and dimension
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (slot[j] < 0) continue;
      const int blk = slot[j] >> 4, off = slot[j] & (kBlock - 1);
      uint8_t* vrow = vp + (((int64_t)blk * KV + kvh) * D + 8 * p) * kBlock + off;
#pragma unroll
      for (int k = 0; k < 8; ++k) vrow[k * kBlock] = (uint8_t)(packed[k] >> (8 * j));
      if (p == 0) sp[((int64_t)blk * KV + kvh) * kBlock + off] = scale[j];
    }
  }

  // K: 16-byte pieces into the page chunk of each token's slot
  if (WITH_K) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (kslot[j] < 0) continue;
      const int blk = kslot[j] >> 4, off = kslot[j] & (kBlock - 1);
      uint16_t* kdst = kp + ((int64_t)blk * KV + kvh) * kBlock * D + (p * kBlock + off) * 8;
      *reinterpret_cast<uint4*>(kdst) = kw[j];
    }
  }

  if (full) {
    // LDS transpose: lane (r, p) holds bytes [r*J, r*J+J) of dimension lines 8p..8p+7
    uint8_t* mine = reinterpret_cast<uint8_t*>(lds_codes[wave]);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint8_t* dst = mine + (8 * p + k) * kBlock + r * J;
      if (J == 4)
        *reinterpret_cast<uint32_t*>(dst) = packed[k];
      else
        *reinterpret_cast<uint16_t*>(dst) = (uint16_t)packed[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t page = (int64_t)(slot0 >> 4) * KV + kvh;
    uint4* vdst = reinterpret_cast<uint4*>(vp + page * D * kBlock);
#pragma unroll
    for (int d = lane; d < D; d += kWave) vdst[d] = lds_codes[wave][d];
    // scales: lane (r, p < J) writes token r*J + p (16 consecutive floats per wave)
    if (p < J) {
      float sc = scale[0];
#pragma unroll
      for (int j = 1; j < J; ++j)
        if (p == j) sc = scale[j];
      sp[page * kBlock + r * J + p] = sc;
    }
  }
}

}  // namespace sdv

using namespace sdv;

static int quant_append(const void* v_new, const void* k_new, const int32_t* slot_mapping, int32_t n_tokens,
                        int32_t kv_heads, int32_t head_dim, int32_t group_size, int32_t num_layers,
                        int64_t in_layer_stride, void* k_pages, void* v_pages, float* v_scales,
                        int32_t num_blocks, int64_t k_layer_stride, int64_t v_layer_stride,
                        int64_t s_layer_stride, int32_t scale_mode, const int32_t* tiles, int32_t n_tiles,
                        void* stream, const SlotTable* table = nullptr) {
  if (!v_new || !(slot_mapping || table) || !v_pages || !v_scales) return SDV_ERR_NULL;
  if (k_new && !k_pages) return SDV_ERR_NULL;
  if (n_tokens < 0 || kv_heads <= 0 || num_layers <= 0 || num_blocks <= 0) return SDV_ERR_SHAPE;
  if (kv_heads > 65535 || num_layers > 65535) return SDV_ERR_SHAPE;
  if (head_dim != 64 && head_dim != 128) return SDV_ERR_UNSUPPORTED;
  if (group_size != head_dim) return SDV_ERR_UNSUPPORTED;
  if (scale_mode != SDV_SCALE_DIV && scale_mode != SDV_SCALE_RCP) return SDV_ERR_UNSUPPORTED;
  const int64_t per_layer_in = (int64_t)n_tokens * kv_heads * head_dim;
  const int64_t k_page = (int64_t)num_blocks * kv_heads * kBlock * head_dim;
  const int64_t s_page = (int64_t)num_blocks * kv_heads * kBlock;
  if (num_layers > 1) {
    if (in_layer_stride < per_layer_in || v_layer_stride < k_page || s_layer_stride < s_page ||
        (k_new && k_layer_stride < k_page))
      return SDV_ERR_SHAPE;
  }
  if (!aligned(v_new, 16) || !aligned(k_new, 16) || !aligned(k_pages, 16) || !aligned(v_pages, 16) ||
      !aligned(v_scales, 4) || !aligned(slot_mapping, 4))
    return SDV_ERR_ALIGN;
  if (num_layers > 1 && (in_layer_stride % 8 != 0 || (k_new && k_layer_stride % 8 != 0)))
    return SDV_ERR_ALIGN;  // 16-byte rows in every layer
  if (n_tokens == 0) return SDV_OK;

  QuantArgs a;
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.slots = slot_mapping;
  a.n_tokens = n_tokens;
  a.kv_heads = kv_heads;
  a.num_blocks = num_blocks;
  a.scale_mode = scale_mode;
  a.in_ls = num_layers > 1 ? in_layer_stride : 0;
  a.k_pages = static_cast<uint16_t*>(k_pages);
  a.v_pages = static_cast<uint8_t*>(v_pages);
  a.v_scales = v_scales;
  a.k_ls = num_layers > 1 ? k_layer_stride : 0;
  a.v_ls = num_layers > 1 ? v_layer_stride : 0;
  a.s_ls = num_layers > 1 ? s_layer_stride : 0;

  a.tiles = tiles;
  a.n_tiles = n_tiles;
  a.table = table ? *table : SlotTable{nullptr, 0, nullptr, 1, 0};
  if (!slot_mapping && (!a.table.block_table || a.table.q_len <= 0 || a.table.max_blocks <= 0)) return SDV_ERR_NULL;

  const int64_t n_waves = tiles ? n_tiles : (n_tokens + kBlock - 1) / kBlock;
  if (n_waves == 0) return SDV_OK;
  dim3 grid((unsigned)((n_waves + kQuantWaves - 1) / kQuantWaves), kv_heads, num_layers);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 block(64 * kQuantWaves);
  if (tiles) {
    if (head_dim == 128 && k_new)
      hipLaunchKernelGGL((quant_append_kernel<128, true, true>), grid, block, 0, st, a);
    else if (head_dim == 128)
      hipLaunchKernelGGL((quant_append_kernel<128, false, true>), grid, block, 0, st, a);
    else if (k_new)
      hipLaunchKernelGGL((quant_append_kernel<64, true, true>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((quant_append_kernel<64, false, true>), grid, block, 0, st, a);
  } else {
    if (head_dim == 128 && k_new)
      hipLaunchKernelGGL((quant_append_kernel<128, true, false>), grid, block, 0, st, a);
    else if (head_dim == 128)
      hipLaunchKernelGGL((quant_append_kernel<128, false, false>), grid, block, 0, st, a);
    else if (k_new)
      hipLaunchKernelGGL((quant_append_kernel<64, true, false>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((quant_append_kernel<64, false, false>), grid, block, 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? SDV_OK : SDV_ERR_HIP;
}

extern "C" int sdv_quant_append(const void* v_new, const void* k_new, const int32_t* slot_mapping,
                                int32_t n_tokens, int32_t kv_heads, int32_t head_dim,
                                int32_t group_size, int32_t num_layers, int64_t in_layer_stride,
                                void* k_pages, void* v_pages, float* v_scales, int32_t num_blocks,
                                int64_t k_layer_stride, int64_t v_layer_stride,
                                int64_t s_layer_stride, int32_t scale_mode, void* stream) {
  return quant_append(v_new, k_new, slot_mapping, n_tokens, kv_heads, head_dim, group_size, num_layers,
                      in_layer_stride, k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride,
                      s_layer_stride, scale_mode, nullptr, 0, stream);
}

extern "C" int sdv_quant_append_tiles(const void* v_new, const void* k_new, const int32_t* slot_mapping,
                                      int32_t n_tokens, int32_t kv_heads, int32_t head_dim,
                                      int32_t group_size, int32_t num_layers, int64_t in_layer_stride,
                                      void* k_pages, void* v_pages, float* v_scales, int32_t num_blocks,
                                      int64_t k_layer_stride, int64_t v_layer_stride,
                                      int64_t s_layer_stride, int32_t scale_mode, const int32_t* tile_starts,
                                      int32_t n_tiles, void* stream) {
  if (!tile_starts) return SDV_ERR_NULL;
  if (n_tiles < 0) return SDV_ERR_SHAPE;
  if (!aligned(tile_starts, 4)) return SDV_ERR_ALIGN;
  return quant_append(v_new, k_new, slot_mapping, n_tokens, kv_heads, head_dim, group_size, num_layers,
                      in_layer_stride, k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride,
                      s_layer_stride, scale_mode, tile_starts, n_tiles, stream);
}

int sdv::quant_append_table(const void* v_new, const void* k_new, const SlotTable& table, int32_t n_tokens,
                            int32_t kv_heads, int32_t head_dim, int32_t num_layers, int64_t in_layer_stride,
                            void* k_pages, void* v_pages, float* v_scales, int32_t num_blocks,
                            int64_t k_layer_stride, int64_t v_layer_stride, int64_t s_layer_stride,
                            int32_t scale_mode, void* stream) {
  return quant_append(v_new, k_new, nullptr, n_tokens, kv_heads, head_dim, head_dim, num_layers, in_layer_stride,
                      k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride, s_layer_stride,
                      scale_mode, nullptr, 0, stream, &table);
}

// Kernel 1: fused V-only FP8 quantize + paged append (and the BF16 K copy).
//
// Restates, per (token, KV head), specdec/engine/model_self.py:304-314 with group_size ==
// head_dim (the v_fp8 format, model_self.py:690,703): s = max|v| / 448 (s == 0 -> 1),
// payload = RNE_E4M3FN(v / s), and the append of payload, scale and BF16 K
// (model_self.py:721-722, 795-799) -- written into pages instead of concatenated.
//
// K is copied into the page's [D/8][16][8] chunk layout (see include/sdv.h).
//
// One wavefront handles 16 consecutive tokens of one KV head of one layer.  Lane l owns
// head_dim/64 adjacent dimensions, so each token's 128-dim row is one coalesced 256-byte
// load and the max-abs is a wave reduction (DPP row rotations + cross-row readlanes).
// When the 16 tokens fill one page block exactly (prefill), each lane accumulates its
// dimensions' 16 codes and writes them with one 16-byte store per dimension (the V page is
// dimension-major); otherwise codes go out as single bytes per slot (decode append).
#include "sdv_internal.h"

namespace sdv {

struct QuantArgs {
  const uint16_t* v_new;
  const uint16_t* k_new;
  const int32_t* slots;
  int n_tokens;
  int kv_heads;
  int num_blocks;
  int scale_mode;
  int64_t in_ls;
  uint16_t* k_pages;
  uint8_t* v_pages;
  float* v_scales;
  int64_t k_ls, v_ls, s_ls;
};

template <int D>
__global__ __launch_bounds__(64) void quant_append_kernel(QuantArgs a) {
  constexpr int DPL = D / 64;  // dimensions per lane
  const int lane = threadIdx.x;
  const int t0 = blockIdx.x * kBlock;
  const int kvh = blockIdx.y;
  const int layer = blockIdx.z;
  const int nt = min(kBlock, a.n_tokens - t0);
  const int KV = a.kv_heads;

  const uint16_t* vin = a.v_new + layer * a.in_ls;
  const uint16_t* kin = a.k_new ? a.k_new + layer * a.in_ls : nullptr;
  uint16_t* kp = a.k_pages + layer * a.k_ls;
  uint8_t* vp = a.v_pages + layer * a.v_ls;
  float* sp = a.v_scales + layer * a.s_ls;

  int my_slot = -1;
  if (lane < nt) {
    my_slot = a.slots[t0 + lane];
    if ((int64_t)my_slot >= (int64_t)a.num_blocks * kBlock) my_slot = -1;  // out-of-range slot: skipped
  }
  const int slot0 = __builtin_amdgcn_readlane(my_slot, 0);
  const uint64_t run = __ballot(lane < kBlock && my_slot == slot0 + lane);
  const bool full = (nt == kBlock) && slot0 >= 0 && (slot0 & (kBlock - 1)) == 0 &&
                    (run & 0xFFFFull) == 0xFFFFull;

  // Issue every token's row load first (16 independent loads in flight).
  uint32_t w[kBlock];
#pragma unroll
  for (int i = 0; i < kBlock; ++i) {
    w[i] = 0;
    if (i < nt) {
      const uint16_t* src = vin + ((int64_t)(t0 + i) * KV + kvh) * D + DPL * lane;
      w[i] = (DPL == 2) ? *reinterpret_cast<const uint32_t*>(src) : (uint32_t)*src;
    }
  }

  uint32_t packed[DPL][4];  // full-block path: 16 codes per owned dimension
#pragma unroll
  for (int d = 0; d < DPL; ++d)
#pragma unroll
    for (int k = 0; k < 4; ++k) packed[d][k] = 0;
  float my_scale = 1.0f;

#pragma unroll
  for (int i = 0; i < kBlock; ++i) {
    const int slot = __builtin_amdgcn_readlane(my_slot, i);  // -1 beyond nt
    if (slot < 0) continue;  // wave-uniform: padding token or past the end
    const float x0 = bf16_lo(w[i]);
    const float x1 = (DPL == 2) ? bf16_hi(w[i]) : 0.0f;
    uint32_t mb = __float_as_uint(fabsf(x0));
    if (DPL == 2) mb = max(mb, __float_as_uint(fabsf(x1)));
    const float amax = __uint_as_float(wave_max_nonneg_bits(mb));
    float s = (a.scale_mode == SDV_SCALE_RCP) ? amax * (1.0f / 448.0f) : amax / 448.0f;
    if (s == 0.0f) s = 1.0f;
    const uint32_t c0 = e4m3fn_encode(x0 / s);
    const uint32_t c1 = (DPL == 2) ? e4m3fn_encode(x1 / s) : 0u;

    const int blk = slot >> 4, off = slot & (kBlock - 1);
    const int64_t page = (int64_t)blk * KV + kvh;
    if (kin) {
      // K page: [D/8 chunks][16 tokens][8 dims]; lane's dims DPL*lane.. sit in chunk DPL*lane/8
      const uint16_t* ksrc = kin + ((int64_t)(t0 + i) * KV + kvh) * D + DPL * lane;
      const int d0 = DPL * lane;
      uint16_t* kdst = kp + page * kBlock * D + ((d0 >> 3) * kBlock + off) * 8 + (d0 & 7);
      if (DPL == 2)
        *reinterpret_cast<uint32_t*>(kdst) = *reinterpret_cast<const uint32_t*>(ksrc);
      else
        *kdst = *ksrc;
    }
    if (full) {
      packed[0][i >> 2] |= c0 << (8 * (i & 3));
      if (DPL == 2) packed[DPL - 1][i >> 2] |= c1 << (8 * (i & 3));
      if (lane == i) my_scale = s;
    } else {
      uint8_t* vrow = vp + (page * D + DPL * lane) * kBlock + off;
      vrow[0] = (uint8_t)c0;
      if (DPL == 2) vrow[kBlock] = (uint8_t)c1;
      if (lane == 0) sp[page * kBlock + off] = s;
    }
  }

  if (full) {
    const int64_t page = (int64_t)(slot0 >> 4) * KV + kvh;
#pragma unroll
    for (int d = 0; d < DPL; ++d) {
      uint4 v4 = make_uint4(packed[d][0], packed[d][1], packed[d][2], packed[d][3]);
      *reinterpret_cast<uint4*>(vp + (page * D + DPL * lane + d) * kBlock) = v4;
    }
    if (lane < kBlock) sp[page * kBlock + lane] = my_scale;
  }
}

}  // namespace sdv

using namespace sdv;

extern "C" int sdv_quant_append(const void* v_new, const void* k_new, const int32_t* slot_mapping,
                                int32_t n_tokens, int32_t kv_heads, int32_t head_dim,
                                int32_t group_size, int32_t num_layers, int64_t in_layer_stride,
                                void* k_pages, void* v_pages, float* v_scales, int32_t num_blocks,
                                int64_t k_layer_stride, int64_t v_layer_stride,
                                int64_t s_layer_stride, int32_t scale_mode, void* stream) {
  if (!v_new || !slot_mapping || !v_pages || !v_scales) return SDV_ERR_NULL;
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
  if (!aligned(v_new, 4) || !aligned(k_new, 4) || !aligned(k_pages, 4) || !aligned(v_pages, 16) ||
      !aligned(v_scales, 4) || !aligned(slot_mapping, 4))
    return SDV_ERR_ALIGN;
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

  dim3 grid((n_tokens + kBlock - 1) / kBlock, kv_heads, num_layers);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    hipLaunchKernelGGL(quant_append_kernel<128>, grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL(quant_append_kernel<64>, grid, dim3(64), 0, st, a);
  return hipGetLastError() == hipSuccess ? SDV_OK : SDV_ERR_HIP;
}

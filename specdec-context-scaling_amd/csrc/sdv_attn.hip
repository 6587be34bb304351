// Kernels 2/3: paged GQA attention over BF16 K and FP8-E4M3 V, decode (q_len = 1) and
// speculative verify (q_len = k+1), with the eager path's rounding points.
//
// The reference computes (specdec/engine/model_self.py:739-776):
//   scores = bf16( bf16(q @ k^T) / sqrt(D) )        -- two BF16 roundings
//   p      = bf16( softmax_fp32(masked scores) )    -- normalised by the GLOBAL max and sum
//   out    = bf16( p @ v_hat ),  v_hat = bf16(fp32(code) * scale)   (model_self.py:316-320)
// Because p is rounded to BF16 after the global normalisation, a one-pass rescaled
// online softmax cannot reproduce it; the work is split in three launches:
//
//   qk_kernel     per (chunk of blocks, KV head, row group, layer*batch): q.k^T on MFMA
//                 (v_mfma_f32_16x16x32_bf16, K rows straight from the page as the A operand,
//                 all query rows of the GQA group as the B operand), BF16 score rounding,
//                 offset-causal mask, BF16 scores to the workspace and the chunk's (max, sum)
//                 from per-lane online statistics merged across the 4 lane groups.
//   pv_kernel     same grid: merges the chunk statistics of its group into the global (M, L),
//                 p = bf16(exp(s - M) / L), dequantises FP8 V in registers
//                 (v_cvt_f32_fp8, fp32 scale multiply, v_cvt_pk_bf16_f32) and accumulates
//                 O^T = V_hat^T P^T on MFMA over pairs of page blocks (32 tokens per MFMA);
//                 the page's dimension-major V layout makes each lane's 4 tokens of one
//                 dimension a single 4-byte load.  fp32 partial O per chunk to the workspace.
//   reduce_kernel sums the partials of each (row, dim) in chunk order (deterministic) and
//                 writes BF16.
//
// MFMA 16x16x32 lane layout (measured on gfx950): A lane l supplies row l%16, B lane l
// supplies column l%16, both with the same 8 k-slots for lane group l/16; the result lane
// l holds rows 4*(l/16)+i, column l%16.  Every operand below uses that mapping.
#include "sdv_internal.h"

namespace sdv {

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k_pages;
  const uint8_t* v_pages;
  const float* v_scales;
  int64_t k_ls, v_ls, s_ls;
  const int32_t* block_table;
  const int32_t* seq_lens;
  uint16_t* out;
  uint16_t* scores;
  float2* stats;
  float* partial;
  int64_t q_ls, q_sb, q_sh, q_ss;  // element strides of q/out: layer, batch, head, row
  int max_blocks, num_blocks, max_seq_len;
  int B, KV, S, G, R;
  int n_row_groups, rpad;
  int chunk_blocks, chunk_tokens, n_chunks, score_stride;
  float sqrt_d;
};

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ bf16x8 zero_bf16x8() { return __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0)); }

__device__ __forceinline__ int seq_len_of(const AttnArgs& a, int b) {
  return min(max(a.seq_lens[b], 0), a.max_seq_len);
}

// ---------------------------------------------------------------------------- q.k^T
template <int D, int NT>
__global__ __launch_bounds__(64) void qk_kernel(AttnArgs a) {
  constexpr int KK = D / 32;  // MFMA k-steps over the head dimension
  constexpr int P = 4;        // page blocks loaded per group of the main loop
  const int lane = threadIdx.x, g = lane >> 4, n = lane & 15;
  const int c = blockIdx.x;
  const int rg = blockIdx.y % a.n_row_groups, kvh = blockIdx.y / a.n_row_groups;
  const int zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int tok0 = c * a.chunk_tokens;
  if (tok0 >= T) return;
  const int grp = zb * a.KV + kvh;

  bf16x8 qop[NT][KK];
  int row[NT], qsi[NT];
  bool rv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    row[nt] = (rg * NT + nt) * 16 + n;
    rv[nt] = row[nt] < a.R;
    const int hl = rv[nt] ? row[nt] / a.S : 0;
    qsi[nt] = rv[nt] ? row[nt] % a.S : 0;
    const uint16_t* qp = a.q + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh +
                         qsi[nt] * a.q_ss + g * 8;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qop[nt][kk] = rv[nt] ? load_bf16x8(qp + kk * 32) : zero_bf16x8();
  }

  const int nblk = min(a.chunk_blocks, (T - tok0 + kBlock - 1) / kBlock);
  int my_pb = -1;
  if (lane < nblk) my_pb = a.block_table[(int64_t)b * a.max_blocks + tok0 / kBlock + lane];
  if (my_pb >= a.num_blocks) my_pb = -1;

  float m_run[NT], l_run[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) { m_run[nt] = -INFINITY; l_run[nt] = 0.0f; }

  const uint16_t* kbase = a.k_pages + layer * a.k_ls + (int64_t)n * D + g * 8;
  for (int j0 = 0; j0 < nblk; j0 += P) {
    bf16x8 kop[P][KK];
    int pbs[P];
#pragma unroll
    for (int u = 0; u < P; ++u) {
      pbs[u] = (j0 + u < nblk) ? __builtin_amdgcn_readlane(my_pb, j0 + u) : -1;
      const uint16_t* kp = kbase + ((int64_t)max(pbs[u], 0) * a.KV + kvh) * (kBlock * D);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kop[u][kk] = (pbs[u] >= 0) ? load_bf16x8(kp + kk * 32) : zero_bf16x8();
    }
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (j0 + u >= nblk) break;
      f32x4 acc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        acc[nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[u][kk], qop[nt][kk], acc[nt], 0, 0, 0);
      }
      const int tb = tok0 + (j0 + u) * kBlock + 4 * g;  // this lane's first token
      const bool blk_ok = pbs[u] >= 0;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float s4[4];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tb + i;
          const float x = round_bf16(round_bf16(acc[nt][i]) / a.sqrt_d);
          const bool vis = blk_ok && t < T && t <= T - a.S + qsi[nt];
          s4[i] = vis ? x : -INFINITY;
          mt = fmaxf(mt, s4[i]);
        }
        if (rv[nt]) {
          uint16_t* sp = a.scores + ((int64_t)grp * a.R + row[nt]) * a.score_stride + tb;
          *reinterpret_cast<uint2*>(sp) = make_uint2(pack_bf16x2(s4[0], s4[1]), pack_bf16x2(s4[2], s4[3]));
        }
        if (mt != -INFINITY) {
          const float mn = fmaxf(m_run[nt], mt);
          float l = (m_run[nt] == -INFINITY) ? 0.0f : l_run[nt] * expf(m_run[nt] - mn);
#pragma unroll
          for (int i = 0; i < 4; ++i) l += expf(s4[i] - mn);
          m_run[nt] = mn;
          l_run[nt] = l;
        }
      }
    }
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float m = m_run[nt], l = l_run[nt];
    merge_stat(m, l, xor_lane(m, 16), xor_lane(l, 16));
    merge_stat(m, l, xor_lane(m, 32), xor_lane(l, 32));
    if (g == 0 && rv[nt]) a.stats[((int64_t)grp * a.n_chunks + c) * a.rpad + row[nt]] = make_float2(m, l);
  }
}

// ---------------------------------------------------------------------------- p.V
template <int D, int NT>
__global__ __launch_bounds__(64) void pv_kernel(AttnArgs a) {
  constexpr int DT = D / 16;  // 16-dimension MFMA tiles
  const int lane = threadIdx.x, g = lane >> 4, n = lane & 15;
  const int c = blockIdx.x;
  const int rg = blockIdx.y % a.n_row_groups, kvh = blockIdx.y / a.n_row_groups;
  const int zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int tok0 = c * a.chunk_tokens;
  if (tok0 >= T) return;
  const int grp = zb * a.KV + kvh;
  const int nvc = (T + a.chunk_tokens - 1) / a.chunk_tokens;

  // Global softmax statistics of this lane's rows (all 4 lane groups end with the same value).
  int row[NT];
  bool rv[NT];
  float gm[NT], ginv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    row[nt] = (rg * NT + nt) * 16 + n;
    rv[nt] = row[nt] < a.R;
    float m = -INFINITY, l = 0.0f;
    if (rv[nt]) {
      const float2* st = a.stats + (int64_t)grp * a.n_chunks * a.rpad + row[nt];
      for (int cc = g; cc < nvc; cc += 4) {
        const float2 v = st[(int64_t)cc * a.rpad];
        merge_stat(m, l, v.x, v.y);
      }
    }
    merge_stat(m, l, xor_lane(m, 16), xor_lane(l, 16));
    merge_stat(m, l, xor_lane(m, 32), xor_lane(l, 32));
    gm[nt] = m;
    ginv[nt] = 1.0f / l;
  }

  const int nblk = min(a.chunk_blocks, (T - tok0 + kBlock - 1) / kBlock);
  int my_pb = -1;
  if (lane < nblk) my_pb = a.block_table[(int64_t)b * a.max_blocks + tok0 / kBlock + lane];
  if (my_pb >= a.num_blocks) my_pb = -1;

  f32x4 acc[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[dt][nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  const uint8_t* vlayer = a.v_pages + layer * a.v_ls;
  const float* slayer = a.v_scales + layer * a.s_ls;
  for (int j = 0; j < nblk; j += 2) {
    const int pb0 = __builtin_amdgcn_readlane(my_pb, j);
    const int pb1 = (j + 1 < nblk) ? __builtin_amdgcn_readlane(my_pb, j + 1) : -1;
    const int tb0 = tok0 + j * kBlock + 4 * g;
    const int tb1 = tb0 + kBlock;
    const bool ok0 = pb0 >= 0, ok1 = pb1 >= 0;

    // this lane's 8 tokens: slots 0..3 = block j tokens 4g..4g+3, slots 4..7 = block j+1
    float4 sc0 = make_float4(0.f, 0.f, 0.f, 0.f), sc1 = sc0;
    if (ok0) sc0 = *reinterpret_cast<const float4*>(slayer + ((int64_t)pb0 * a.KV + kvh) * kBlock + 4 * g);
    if (ok1) sc1 = *reinterpret_cast<const float4*>(slayer + ((int64_t)pb1 * a.KV + kvh) * kBlock + 4 * g);
    uint32_t w0[DT], w1[DT];
    const uint8_t* vp0 = vlayer + (((int64_t)max(pb0, 0) * a.KV + kvh) * D + n) * kBlock + 4 * g;
    const uint8_t* vp1 = vlayer + (((int64_t)max(pb1, 0) * a.KV + kvh) * D + n) * kBlock + 4 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      w0[dt] = ok0 ? *reinterpret_cast<const uint32_t*>(vp0 + dt * 16 * kBlock) : 0u;
      w1[dt] = ok1 ? *reinterpret_cast<const uint32_t*>(vp1 + dt * 16 * kBlock) : 0u;
    }

    bool tv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tv[i] = ok0 && (tb0 + i < T);
      tv[4 + i] = ok1 && (tb1 + i < T);
    }

    // P^T operands (B): probabilities of this lane's row for its 8 tokens.
    bf16x8 pop[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      uint32_t pw[4] = {0u, 0u, 0u, 0u};
      if (rv[nt]) {
        const uint16_t* sp = a.scores + ((int64_t)grp * a.R + row[nt]) * a.score_stride;
        uint2 s0 = make_uint2(0xFF80FF80u, 0xFF80FF80u), s1 = s0;  // -inf pairs
        if (ok0) s0 = *reinterpret_cast<const uint2*>(sp + tb0);
        if (ok1) s1 = *reinterpret_cast<const uint2*>(sp + tb1);
        const uint32_t sw[4] = {s0.x, s0.y, s1.x, s1.y};
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float s = (i & 1) ? bf16_hi(sw[i >> 1]) : bf16_lo(sw[i >> 1]);
          p[i] = tv[i] ? round_bf16(expf(s - gm[nt]) * ginv[nt]) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) pw[k] = pack_bf16x2(p[2 * k], p[2 * k + 1]);
      }
      pop[nt] = __builtin_bit_cast(bf16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
    }

    const float scl[8] = {sc0.x, sc0.y, sc0.z, sc0.w, sc1.x, sc1.y, sc1.z, sc1.w};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      // V_hat^T operand (A): dimension dt*16+n, the same 8 tokens.
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = tv[i] ? round_bf16(e4m3fn_decode(w0[dt], i) * scl[i]) : 0.0f;
        v[4 + i] = tv[4 + i] ? round_bf16(e4m3fn_decode(w1[dt], i) * scl[4 + i]) : 0.0f;
      }
      const bf16x8 vop = __builtin_bit_cast(
          bf16x8, make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                             pack_bf16x2(v[6], v[7])));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[nt], acc[dt][nt], 0, 0, 0);
    }
  }

  // lane (g, n) holds O^T[dims dt*16 + 4g .. +3][row n]
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if (!rv[nt]) continue;
    float* dst = a.partial + (((int64_t)grp * a.n_chunks + c) * a.R + row[nt]) * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<float4*>(dst + dt * 16) =
          make_float4(acc[dt][nt][0], acc[dt][nt][1], acc[dt][nt][2], acc[dt][nt][3]);
  }
}

// ---------------------------------------------------------------------------- reduce
template <int D>
__global__ __launch_bounds__(256) void reduce_kernel(AttnArgs a) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int kvh = blockIdx.y;
  const int zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  if (idx >= a.R * D) return;
  const int r = idx / D, d = idx % D;
  const int T = seq_len_of(a, b);
  const int nvc = (T + a.chunk_tokens - 1) / a.chunk_tokens;
  const int grp = zb * a.KV + kvh;
  const float* src = a.partial + ((int64_t)grp * a.n_chunks * a.R + r) * D + d;
  const int64_t step = (int64_t)a.R * D;
  float sum = 0.0f;
  for (int cc = 0; cc < nvc; ++cc) sum += src[cc * step];
  const int hl = r / a.S, si = r % a.S;
  uint16_t* o = a.out + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + d;
  *o = (uint16_t)bf16_bits(sum);
}

// ---------------------------------------------------------------------------- planning
struct Plan {
  int NT, n_row_groups, rpad;
  int chunk_blocks, chunk_tokens, n_chunks, score_stride;
  size_t off_stats, off_partial, total;
};

static bool make_plan(int L, int B, int H, int KV, int S, int D, int max_seq_len, Plan* p) {
  if (L <= 0 || B <= 0 || H <= 0 || KV <= 0 || S <= 0 || max_seq_len <= 0) return false;
  if (H % KV) return false;
  if (L > 65535 || (int64_t)L * B > 65535) return false;
  const int G = H / KV;
  const int64_t R = (int64_t)G * S;
  if (R > (1 << 20)) return false;
  p->NT = R <= 16 ? 1 : R <= 32 ? 2 : R <= 48 ? 3 : 4;
  p->n_row_groups = (int)((R + 16 * p->NT - 1) / (16 * p->NT));
  if ((int64_t)KV * p->n_row_groups > 65535) return false;
  p->rpad = p->n_row_groups * p->NT * 16;
  // Chunk size: enough workgroups to cover the 256 CUs several times over, chunks of at
  // least two page blocks (the PV MFMA consumes 32 tokens) and at most 32 blocks.
  const int64_t total_blocks = (int64_t)L * B * KV * ((max_seq_len + kBlock - 1) / kBlock);
  int cb = 2;
  while (cb < 32 && total_blocks / (2 * cb) >= 2048) cb *= 2;
  p->chunk_blocks = cb;
  p->chunk_tokens = cb * kBlock;
  p->n_chunks = (max_seq_len + p->chunk_tokens - 1) / p->chunk_tokens;
  p->score_stride = p->n_chunks * p->chunk_tokens;
  const int64_t groups = (int64_t)L * B * KV;
  const size_t scores = round_up((size_t)(groups * R * p->score_stride * 2), 256);
  const size_t stats = round_up((size_t)(groups * p->n_chunks * p->rpad * 8), 256);
  const size_t partial = round_up((size_t)(groups * p->n_chunks * R * D * 4), 256);
  p->off_stats = scores;
  p->off_partial = scores + stats;
  p->total = scores + stats + partial;
  return true;
}

template <int D, int NT>
static void launch_qk_pv(const AttnArgs& a, dim3 grid, hipStream_t st, int phases) {
  if (phases & SDV_PHASE_QK) hipLaunchKernelGGL((qk_kernel<D, NT>), grid, dim3(64), 0, st, a);
  if (phases & SDV_PHASE_PV) hipLaunchKernelGGL((pv_kernel<D, NT>), grid, dim3(64), 0, st, a);
}

template <int D>
static void launch_all(const AttnArgs& a, const Plan& p, int layers_x_batch, hipStream_t st, int phases) {
  const dim3 grid(p.n_chunks, a.KV * p.n_row_groups, layers_x_batch);
  switch (p.NT) {
    case 1: launch_qk_pv<D, 1>(a, grid, st, phases); break;
    case 2: launch_qk_pv<D, 2>(a, grid, st, phases); break;
    case 3: launch_qk_pv<D, 3>(a, grid, st, phases); break;
    default: launch_qk_pv<D, 4>(a, grid, st, phases); break;
  }
  if (phases & SDV_PHASE_REDUCE)
    hipLaunchKernelGGL(reduce_kernel<D>, dim3((a.R * D + 255) / 256, a.KV, layers_x_batch), dim3(256), 0, st, a);
}

}  // namespace sdv

using namespace sdv;

extern "C" size_t sdv_attention_workspace_size(int32_t num_layers, int32_t batch, int32_t q_heads,
                                               int32_t kv_heads, int32_t q_len, int32_t head_dim,
                                               int32_t max_seq_len) {
  if (head_dim != 64 && head_dim != 128) return 0;
  Plan p;
  if (!make_plan(num_layers, batch, q_heads, kv_heads, q_len, head_dim, max_seq_len, &p)) return 0;
  return p.total;
}

extern "C" int sdv_paged_attention_phases(const void* q, const void* k_pages, const void* v_pages,
                                          const float* v_scales, int32_t num_blocks, int64_t k_layer_stride,
                                          int64_t v_layer_stride, int64_t s_layer_stride,
                                          const int32_t* block_table, int32_t max_blocks_per_seq,
                                          const int32_t* seq_lens, int32_t num_layers, int32_t batch,
                                          int32_t q_heads, int32_t kv_heads, int32_t q_len, int32_t head_dim,
                                          int32_t max_seq_len, int32_t q_token_major, void* workspace,
                                          size_t workspace_bytes, void* out, void* stream, int32_t phase_mask) {
  if (phase_mask <= 0 || phase_mask > SDV_PHASE_ALL) return SDV_ERR_SHAPE;
  if (!q || !k_pages || !v_pages || !v_scales || !block_table || !seq_lens || !out) return SDV_ERR_NULL;
  if (head_dim != 64 && head_dim != 128) return SDV_ERR_UNSUPPORTED;
  if (num_blocks <= 0 || max_blocks_per_seq <= 0) return SDV_ERR_SHAPE;
  if (q_token_major != 0 && q_token_major != 1) return SDV_ERR_SHAPE;
  Plan p;
  if (!make_plan(num_layers, batch, q_heads, kv_heads, q_len, head_dim, max_seq_len, &p)) return SDV_ERR_SHAPE;
  if ((int64_t)max_blocks_per_seq * kBlock < max_seq_len) return SDV_ERR_SHAPE;
  const int64_t k_page = (int64_t)num_blocks * kv_heads * kBlock * head_dim;
  const int64_t s_page = (int64_t)num_blocks * kv_heads * kBlock;
  if (num_layers > 1 && (k_layer_stride < k_page || v_layer_stride < k_page || s_layer_stride < s_page))
    return SDV_ERR_SHAPE;
  if (!workspace || workspace_bytes < p.total || !aligned(workspace, 256)) return SDV_ERR_WORKSPACE;
  if (!aligned(q, 16) || !aligned(out, 16) || !aligned(k_pages, 16) || !aligned(v_scales, 16) ||
      !aligned(v_pages, 4) || !aligned(block_table, 4) || !aligned(seq_lens, 4))
    return SDV_ERR_ALIGN;
  if (num_layers > 1 && ((k_layer_stride % 8) || (v_layer_stride % 16) || (s_layer_stride % 4)))
    return SDV_ERR_ALIGN;

  AttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_pages = static_cast<const uint16_t*>(k_pages);
  a.v_pages = static_cast<const uint8_t*>(v_pages);
  a.v_scales = v_scales;
  a.k_ls = num_layers > 1 ? k_layer_stride : 0;
  a.v_ls = num_layers > 1 ? v_layer_stride : 0;
  a.s_ls = num_layers > 1 ? s_layer_stride : 0;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.out = static_cast<uint16_t*>(out);
  char* ws = static_cast<char*>(workspace);
  a.scores = reinterpret_cast<uint16_t*>(ws);
  a.stats = reinterpret_cast<float2*>(ws + p.off_stats);
  a.partial = reinterpret_cast<float*>(ws + p.off_partial);
  const int64_t D = head_dim, S = q_len, H = q_heads;
  a.q_sb = H * S * D;
  a.q_ls = (int64_t)batch * a.q_sb;
  if (q_token_major) {
    a.q_sh = D;
    a.q_ss = H * D;
  } else {
    a.q_sh = S * D;
    a.q_ss = D;
  }
  a.max_blocks = max_blocks_per_seq;
  a.num_blocks = num_blocks;
  a.max_seq_len = max_seq_len;
  a.B = batch;
  a.KV = kv_heads;
  a.S = q_len;
  a.G = q_heads / kv_heads;
  a.R = a.G * q_len;
  a.n_row_groups = p.n_row_groups;
  a.rpad = p.rpad;
  a.chunk_blocks = p.chunk_blocks;
  a.chunk_tokens = p.chunk_tokens;
  a.n_chunks = p.n_chunks;
  a.score_stride = p.score_stride;
  a.sqrt_d = head_dim == 128 ? 11.313708498984761f : 8.0f;

  hipStream_t st = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    launch_all<128>(a, p, num_layers * batch, st, phase_mask);
  else
    launch_all<64>(a, p, num_layers * batch, st, phase_mask);
  return hipGetLastError() == hipSuccess ? SDV_OK : SDV_ERR_HIP;
}

extern "C" int sdv_paged_attention(const void* q, const void* k_pages, const void* v_pages,
                                   const float* v_scales, int32_t num_blocks, int64_t k_layer_stride,
                                   int64_t v_layer_stride, int64_t s_layer_stride,
                                   const int32_t* block_table, int32_t max_blocks_per_seq,
                                   const int32_t* seq_lens, int32_t num_layers, int32_t batch,
                                   int32_t q_heads, int32_t kv_heads, int32_t q_len, int32_t head_dim,
                                   int32_t max_seq_len, int32_t q_token_major, void* workspace,
                                   size_t workspace_bytes, void* out, void* stream) {
  return sdv_paged_attention_phases(q, k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride,
                                    s_layer_stride, block_table, max_blocks_per_seq, seq_lens, num_layers, batch,
                                    q_heads, kv_heads, q_len, head_dim, max_seq_len, q_token_major, workspace,
                                    workspace_bytes, out, stream, SDV_PHASE_ALL);
}

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
//   qk_kernel     workgroup = 4 wavefronts = one chunk of page blocks of one (layer*batch,
//                 KV head, query-row group).  Each wave runs q.k^T on MFMA
//                 (v_mfma_f32_16x16x32_bf16; K rows straight from the page are the A operand,
//                 all query rows of the GQA group the B operand), rounds scores to BF16,
//                 applies the offset-causal mask, writes BF16 scores to the workspace and
//                 keeps online (max, sum) per row; the 4 waves' statistics merge in LDS into
//                 one (max, sum) per chunk.
//   pv_kernel     workgroup = 4 wavefronts = one (larger) chunk.  The 256 threads merge the
//                 group's chunk statistics into the global (M, 1/L) per row (fixed order, via
//                 LDS); each wave computes p = bf16(exp(s - M) / L), dequantises FP8 V in
//                 registers (v_cvt_pk_f32_fp8, fp32 scale multiply, v_cvt_pk_bf16_f32) and
//                 accumulates O^T = V_hat^T P^T on MFMA over pairs of page blocks (32 tokens per
//                 MFMA: the page's dimension-major V layout makes each lane's 4 tokens of one
//                 dimension one 4-byte load); the 4 waves' fp32 partial O sum in LDS.
//   reduce_kernel 64 outputs x 4 chunk slices per workgroup: sums the chunk partials in a
//                 fixed order (deterministic) and writes BF16.
//
// MFMA 16x16x32 lane layout (measured on gfx950): A lane l supplies row l%16, B lane l
// supplies column l%16, both with the same 8 k-slots for lane group l/16; the result lane
// l holds rows 4*(l/16)+i, column l%16.  Every operand below uses that mapping.
#include "sdv_internal.h"

namespace sdv {

constexpr int kWaves = 4;          // wavefronts per workgroup in qk/pv
constexpr int kQkScoreTokens = 128;  // tokens x row tiles of scores one qk wave stages in LDS

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
  int qk_bpw, qk_chunk_tokens, n_qk_chunks;
  int pv_bpw, pv_chunk_tokens, n_pv_chunks;
  int score_stride;
  float inv_sqrt_d;
};

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ bf16x8 zero_bf16x8() { return __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0)); }

__device__ __forceinline__ int seq_len_of(const AttnArgs& a, int b) {
  return min(max(a.seq_lens[b], 0), a.max_seq_len);
}

// exp(x) as 2^(x * log2 e) on v_exp_f32.  The rounding of x * log2 e costs at most
// |x| * 2^-24 relative, far below one BF16 step of the probabilities it feeds (and below
// the fp32 summation noise of L); exp(-inf) = 0.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

__device__ __forceinline__ void merge_fast(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  const float a = (m == -INFINITY) ? 0.0f : l * fast_exp(m - mn);
  const float b = (m2 == -INFINITY) ? 0.0f : l2 * fast_exp(m2 - mn);
  m = mn;
  l = a + b;
}

// ---------------------------------------------------------------------------- q.k^T
template <int D, int NT>
__global__ __launch_bounds__(256) void qk_kernel(AttnArgs a) {
  constexpr int KK = D / 32;  // MFMA k-steps over the head dimension
  constexpr int P = 2;        // page blocks per pipeline stage
  constexpr int SCT = kQkScoreTokens / NT;  // score tokens per row a wave can stage in LDS
  __shared__ float2 lstat[kWaves][NT * 16];
  __shared__ uint2 lsc[kWaves][NT * 16][SCT / 4];  // BF16 scores, 4 tokens per entry
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int c = blockIdx.x;
  const int rg = blockIdx.y % a.n_row_groups, kvh = blockIdx.y / a.n_row_groups;
  const int zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int tok0 = c * a.qk_chunk_tokens;
  if (tok0 >= T) return;  // workgroup-uniform
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

  const int blk0 = (tok0 >> 4) + wave * a.qk_bpw;  // this wave's first block of the sequence
  const int nb = max(0, min(a.qk_bpw, ((T + kBlock - 1) >> 4) - blk0));
  int my_pb = -1;
  if (lane < nb) my_pb = a.block_table[(int64_t)b * a.max_blocks + blk0 + lane];
  if (my_pb >= a.num_blocks) my_pb = -1;

  float m_run[NT], l_run[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) { m_run[nt] = -INFINITY; l_run[nt] = 0.0f; }

  // K page layout [D/8][16][8]: for MFMA step kk, lane l's 16 bytes (token l%16, dims
  // (4kk + l/16)*8 ..) sit at element kk*512 + l*8 -- one contiguous 1 KiB load per step.
  const uint16_t* kbase = a.k_pages + layer * a.k_ls + (int64_t)lane * 8;
  // Two page blocks per pipeline stage: the loads of stage j+1 are in flight while stage j
  // is multiplied, so each wavefront keeps streaming K.
  auto load_stage = [&](int j0, bf16x8 (&kop)[P][KK], int (&pbs)[P]) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      pbs[u] = (j0 + u < nb) ? __builtin_amdgcn_readlane(my_pb, j0 + u) : -1;
      const uint16_t* kp = kbase + ((int64_t)max(pbs[u], 0) * a.KV + kvh) * (kBlock * D);
      // Unconditional loads keep the wait counters exact; a missing or invalid block reads
      // block 0 (always allocated) and its tokens are masked below.
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kop[u][kk] = __builtin_bit_cast(bf16x8, load_stream16(kp + kk * 512));
    }
  };
  auto compute_stage = [&](const bf16x8 (&kop)[P][KK], const int (&pbs)[P], int j0) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (j0 + u >= nb) break;
      f32x4 acc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        acc[nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[u][kk], qop[nt][kk], acc[nt], 0, 0, 0);
      }
      const int tb = (blk0 + j0 + u) * kBlock + 4 * g;  // this lane's first token
      const bool blk_ok = pbs[u] >= 0;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float s4[4];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tb + i;
          // bf16(bf16(q.k) / sqrt(D)): for BF16 inputs, dividing by RN(sqrt(D)) and
          // multiplying by RN(1/sqrt(D)) round to the same BF16 (checked for all inputs).
          const float x = round_bf16(round_bf16(acc[nt][i]) * a.inv_sqrt_d);
          const bool vis = blk_ok && t < T && t <= T - a.S + qsi[nt];
          s4[i] = vis ? x : -INFINITY;
          mt = fmaxf(mt, s4[i]);
        }
        // staged in LDS: global stores mixed with the in-flight K loads would force full waits
        lsc[wave][nt * 16 + n][(j0 + u) * 4 + g] =
            make_uint2(pack_bf16x2(s4[0], s4[1]), pack_bf16x2(s4[2], s4[3]));
        if (mt != -INFINITY) {
          const float mn = fmaxf(m_run[nt], mt);
          float l = (m_run[nt] == -INFINITY) ? 0.0f : l_run[nt] * fast_exp(m_run[nt] - mn);
#pragma unroll
          for (int i = 0; i < 4; ++i) l += fast_exp(s4[i] - mn);
          m_run[nt] = mn;
          l_run[nt] = l;
        }
      }
    }
  };
  // Ping-pong buffers: stage j+1 loads into the other buffer while stage j is computed;
  // no register copies between stages, so a stage's wait covers only its own loads.
  bf16x8 ka[P][KK], kb[P][KK];
  int pa[P], pbb[P];
  // The prefetch is unconditional (a stage past the end reads block 0, which every wave of
  // the layer shares in L2, and is masked): conditional loads would make the wait counters
  // at the loop head imprecise and serialize the pipeline.
  if (nb > 0) load_stage(0, ka, pa);
  for (int j0 = 0; j0 < nb; j0 += 2 * P) {
    load_stage(j0 + P, kb, pbb);
    compute_stage(ka, pa, j0);
    if (j0 + P >= nb) break;
    load_stage(j0 + 2 * P, ka, pa);
    compute_stage(kb, pbb, j0 + P);
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float m = m_run[nt], l = l_run[nt];
    merge_fast(m, l, xor_lane(m, 16), xor_lane(l, 16));
    merge_fast(m, l, xor_lane(m, 32), xor_lane(l, 32));
    if (g == 0) lstat[wave][nt * 16 + n] = make_float2(m, l);
  }
  __syncthreads();
  // This wave's staged scores -> workspace rows, 16 bytes per lane per store (after the
  // barrier: lanes read entries other lanes wrote).
  {
    const int per_row = nb * 2;  // 16-byte pieces per row (16 tokens = 32 bytes per block)
    for (int e = lane; e < NT * 16 * per_row; e += kWave) {
      const int lr = e / per_row, piece = e % per_row;
      const int r = rg * NT * 16 + lr;
      if (r < a.R) {
        const uint2 x0 = lsc[wave][lr][piece * 2], x1 = lsc[wave][lr][piece * 2 + 1];
        uint16_t* sp = a.scores + ((int64_t)grp * a.R + r) * a.score_stride + blk0 * kBlock + piece * 8;
        *reinterpret_cast<uint4*>(sp) = make_uint4(x0.x, x0.y, x1.x, x1.y);
      }
    }
  }
  if (tid < NT * 16) {
    const int r = rg * NT * 16 + tid;
    float m = lstat[0][tid].x, l = lstat[0][tid].y;
#pragma unroll
    for (int w = 1; w < kWaves; ++w) merge_fast(m, l, lstat[w][tid].x, lstat[w][tid].y);
    if (r < a.R) a.stats[((int64_t)grp * a.n_qk_chunks + c) * a.rpad + r] = make_float2(m, l);
  }
}

// ---------------------------------------------------------------------------- p.V
// One PV pipeline stage: 4 page blocks (64 tokens) of one wavefront.  Lane (g, n) owns block
// g of the stage: all 16 tokens of V dimension dt*16+n (one 16-byte load per dimension
// tile; the V page is dimension-major), the 16 scales of the block, and the 16 BF16 scores
// of its query row n.  The MFMA k-slots of lane group g are tokens 8h..8h+7 of block g,
// for the two token halves h.
template <int D, int NT>
struct PvStage {
  uint4 code[D / 16];  // E4M3FN codes, token i of the block in byte i
  float4 scl[4];       // per-token scales
  uint4 sc[NT][2];     // BF16 scores, tokens 0..7 and 8..15
  int blk;             // block index within the sequence (this lane group's)
  bool ok;             // the block exists and its page id is valid
};

template <int D, int NT>
__device__ __forceinline__ void pv_load(PvStage<D, NT>& st, const AttnArgs& a, int j, int my_pb, int nb, int blk0,
                                        const uint8_t* vlayer, const float* slayer, const uint16_t* srow0,
                                        const int64_t (&srow_off)[NT], int kvh, int g, int n) {
  constexpr int DT = D / 16;
  // page id of block j+g (lane-varying): fetched from lane j+g of my_pb
  const int jj = j + g;
  const int pb = __shfl(my_pb, jj < kWave ? jj : 0);
  st.ok = (jj < nb) && (pb >= 0);
  st.blk = blk0 + jj;
  // Unconditional loads keep the wait counters exact: a missing or invalid block reads
  // block 0 (always allocated); its tokens are masked in pv_compute.
  const int64_t page = (int64_t)(st.ok ? pb : 0) * a.KV + kvh;
  const uint8_t* vp = vlayer + (page * D + n) * kBlock;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) st.code[dt] = load_stream16(vp + dt * 16 * kBlock);
  const float* sp = slayer + page * kBlock;
#pragma unroll
  for (int q = 0; q < 4; ++q) st.scl[q] = __builtin_bit_cast(float4, load_stream16(sp + 4 * q));
  // scores of a block past the chunk stay inside the workspace row (score_stride covers it)
  const int64_t tok = (int64_t)min(st.blk, a.score_stride / kBlock - 1) * kBlock;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const uint4* ps = reinterpret_cast<const uint4*>(srow0 + srow_off[nt] + tok);
    st.sc[nt][0] = ps[0];
    st.sc[nt][1] = ps[1];
  }
}

template <int D, int NT>
__device__ __forceinline__ void pv_compute(PvStage<D, NT>& st, f32x4 (&acc)[D / 16][NT], const float (&gm)[NT],
                                           const float (&ginv)[NT], int T, bool stage_full) {
  constexpr int DT = D / 16;
  // wave-uniform: every block of the stage exists, has a valid page and lies below T
  if (!stage_full || __ballot(!st.ok) != 0) {
    // Sanitize the slots that are not tokens of the sequence: codes and scales to 0 (so
    // no NaN pattern of an unwritten page can reach the MFMA), scores to -inf (p = 0).
    const int nvalid = st.ok ? min(max(T - st.blk * kBlock, 0), kBlock) : 0;  // lane-group value
    uint32_t bmask[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int k = min(max(nvalid - 4 * w, 0), 4);  // valid bytes in this word
      bmask[w] = k >= 4 ? 0xFFFFFFFFu : ((1u << (8 * k)) - 1u);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      st.code[dt].x &= bmask[0];
      st.code[dt].y &= bmask[1];
      st.code[dt].z &= bmask[2];
      st.code[dt].w &= bmask[3];
    }
    float* sf = reinterpret_cast<float*>(st.scl);
#pragma unroll
    for (int i = 0; i < 16; ++i) sf[i] = i < nvalid ? sf[i] : 0.0f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      uint32_t* sw = reinterpret_cast<uint32_t*>(st.sc[nt]);
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const uint32_t keep = (2 * w + 1 < nvalid) ? 0xFFFFFFFFu : (2 * w < nvalid ? 0x0000FFFFu : 0u);
        sw[w] = (sw[w] & keep) | (0xFF80FF80u & ~keep);
      }
    }
  }
  const float* sf = reinterpret_cast<const float*>(st.scl);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // P^T operand (B): probabilities of this lane's row for tokens 8h..8h+7 of its block.
    bf16x8 pop[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint4 w4 = st.sc[nt][h];
      const uint32_t sw[4] = {w4.x, w4.y, w4.z, w4.w};
      float pr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float s = (i & 1) ? bf16_hi(sw[i >> 1]) : bf16_lo(sw[i >> 1]);
        pr[i] = fast_exp(s - gm[nt]) * ginv[nt];  // -inf score -> 0
      }
      pop[nt] = __builtin_bit_cast(bf16x8, make_uint4(pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                                                      pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])));
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      // V_hat^T operand (A): dimension dt*16+n, tokens 8h..8h+7 of this lane group's block.
      typedef float f32x2 __attribute__((ext_vector_type(2)));
      const uint32_t lo = h ? st.code[dt].z : st.code[dt].x;
      const uint32_t hi = h ? st.code[dt].w : st.code[dt].y;
      const f32x2 f01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
      const f32x2 f23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
      const f32x2 f45 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
      const f32x2 f67 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
      const float* sc = sf + 8 * h;
      const bf16x8 vop = __builtin_bit_cast(
          bf16x8, make_uint4(pack_bf16x2(f01.x * sc[0], f01.y * sc[1]), pack_bf16x2(f23.x * sc[2], f23.y * sc[3]),
                             pack_bf16x2(f45.x * sc[4], f45.y * sc[5]), pack_bf16x2(f67.x * sc[6], f67.y * sc[7])));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[nt], acc[dt][nt], 0, 0, 0);
    }
  }
}

template <int D, int NT>
__global__ __launch_bounds__(256) void pv_kernel(AttnArgs a) {
  constexpr int DT = D / 16;  // 16-dimension MFMA tiles
  constexpr int RT = NT * 16;
  constexpr int SLICES = 256 / RT;
  __shared__ float2 lstat[SLICES * RT];
  __shared__ float2 lms[RT];
  __shared__ float lacc[kWaves][16][D + 4];  // +4: spread the lane groups over LDS banks
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int c = blockIdx.x;
  const int rg = blockIdx.y % a.n_row_groups, kvh = blockIdx.y / a.n_row_groups;
  const int zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int tok0 = c * a.pv_chunk_tokens;
  if (tok0 >= T) return;  // workgroup-uniform
  const int grp = zb * a.KV + kvh;

  const int blk0 = (tok0 >> 4) + wave * a.pv_bpw;
  const int nb = max(0, min(a.pv_bpw, ((T + kBlock - 1) >> 4) - blk0));
  int my_pb = -1;
  if (lane < nb) my_pb = a.block_table[(int64_t)b * a.max_blocks + blk0 + lane];
  if (my_pb >= a.num_blocks) my_pb = -1;

  // score rows of this lane's query row in each row tile (padding rows read row 0; their
  // MFMA columns are never stored)
  int64_t srow_off[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = rg * RT + nt * 16 + n;
    srow_off[nt] = (int64_t)(r < a.R ? r : 0) * a.score_stride;
  }
  const uint16_t* srow0 = a.scores + (int64_t)grp * a.R * a.score_stride;
  const uint8_t* vlayer = a.v_pages + layer * a.v_ls;
  const float* slayer = a.v_scales + layer * a.s_ls;

  // Stage 0 of V is in flight while the statistics below are merged.
  const int nst = (nb + 3) >> 2;
  PvStage<D, NT> sa, sb;
  if (nst > 0) pv_load<D, NT>(sa, a, 0, my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);

  // --- global softmax statistics of this row group: thread (slice, row) merges chunks
  // slice, slice+SLICES, ...; slices then merge in order.  Fixed order: deterministic.
  {
    const int r = tid % RT, slice = tid / RT;
    const int nvq = (T + a.qk_chunk_tokens - 1) / a.qk_chunk_tokens;
    float m = -INFINITY, l = 0.0f;
    const int srow = rg * RT + r;
    if (slice < SLICES && srow < a.R) {
      const float2* st = a.stats + (int64_t)grp * a.n_qk_chunks * a.rpad + srow;
      int cc = slice;
      for (; cc + 3 * SLICES < nvq; cc += 4 * SLICES) {
        float2 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = st[(int64_t)(cc + u * SLICES) * a.rpad];
#pragma unroll
        for (int u = 0; u < 4; ++u) merge_fast(m, l, v[u].x, v[u].y);
      }
      for (; cc < nvq; cc += SLICES) {
        const float2 v = st[(int64_t)cc * a.rpad];
        merge_fast(m, l, v.x, v.y);
      }
    }
    if (slice < SLICES) lstat[slice * RT + r] = make_float2(m, l);
    __syncthreads();
    if (tid < RT) {
      float mm = lstat[tid].x, ll = lstat[tid].y;
      for (int s2 = 1; s2 < SLICES; ++s2) merge_fast(mm, ll, lstat[s2 * RT + tid].x, lstat[s2 * RT + tid].y);
      lms[tid] = make_float2(mm, 1.0f / ll);
    }
    __syncthreads();
  }
  float gm[NT], ginv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    gm[nt] = lms[nt * 16 + n].x;
    ginv[nt] = lms[nt * 16 + n].y;
  }

  f32x4 acc[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[dt][nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // Ping-pong over stages; the prefetch is unconditional (a stage past the end reads block
  // 0 and is masked) so the wait counters stay exact.  A stage is "full" (no masking) when
  // all 64 of its slots are tokens of the sequence -- wave-uniform.
  const int full_stages = min(nb, max(0, (T >> 4) - blk0)) >> 2;
  int st_i = 0;
  for (; st_i + 1 < nst; st_i += 2) {
    pv_load<D, NT>(sb, a, 4 * (st_i + 1), my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);
    pv_compute<D, NT>(sa, acc, gm, ginv, T, st_i < full_stages);
    pv_load<D, NT>(sa, a, 4 * (st_i + 2), my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);
    pv_compute<D, NT>(sb, acc, gm, ginv, T, st_i + 1 < full_stages);
  }
  if (st_i < nst) pv_compute<D, NT>(sa, acc, gm, ginv, T, st_i < full_stages);

  // lane (g, n) holds O^T[dims dt*16 + 4g .. +3][row n]; the 4 waves sum in LDS per row tile.
  float* dst = a.partial + ((int64_t)grp * a.n_pv_chunks + c) * a.R * D;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) lacc[wave][n][dt * 16 + 4 * g + i] = acc[dt][nt][i];
    __syncthreads();
    for (int e = tid; e < 16 * D; e += 256) {
      const int r = e / D, d = e % D;
      const int rr = rg * RT + nt * 16 + r;
      const float sum = ((lacc[0][r][d] + lacc[1][r][d]) + lacc[2][r][d]) + lacc[3][r][d];
      if (rr < a.R) dst[(int64_t)rr * D + d] = sum;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------- reduce
template <int D>
__global__ __launch_bounds__(256) void reduce_kernel(AttnArgs a) {
  __shared__ float lsum[4][64];
  const int tid = threadIdx.x, o = blockIdx.x * 64 + (tid & 63), slice = tid >> 6;
  const int kvh = blockIdx.y;
  const int zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int nvp = (T + a.pv_chunk_tokens - 1) / a.pv_chunk_tokens;
  const int grp = zb * a.KV + kvh;
  const bool valid = o < a.R * D;
  const int per = (nvp + 3) / 4;
  const int c_lo = slice * per, c_hi = min(nvp, c_lo + per);
  float s = 0.0f;
  if (valid) {
    const float* src = a.partial + (int64_t)grp * a.n_pv_chunks * a.R * D + o;
    const int64_t step = (int64_t)a.R * D;
    int cc = c_lo;
    for (; cc + 8 <= c_hi; cc += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[(cc + u) * step];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; cc < c_hi; ++cc) s += src[cc * step];
  }
  lsum[slice][tid & 63] = s;
  __syncthreads();
  if (slice == 0 && valid) {
    const float sum = ((lsum[0][tid] + lsum[1][tid]) + lsum[2][tid]) + lsum[3][tid];
    const int r = o / D, d = o % D;
    const int hl = r / a.S, si = r % a.S;
    uint16_t* dstp = a.out + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + d;
    *dstp = (uint16_t)bf16_bits(sum);
  }
}

// ---------------------------------------------------------------------------- planning
struct Plan {
  int NT, n_row_groups, rpad;
  int qk_bpw, qk_chunk_tokens, n_qk_chunks;
  int pv_bpw, pv_chunk_tokens, n_pv_chunks;
  int score_stride;
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
  // Chunking over the page blocks of all (layer, sequence, KV head, row group) units.  PV
  // (one third of the bytes) uses chunks twice as long as QK, so fewer fp32 partials are
  // written and reduced.
  const int64_t units = (int64_t)L * B * KV * p->n_row_groups;
  const int64_t blocks = units * ((max_seq_len + kBlock - 1) / kBlock);
  // About one resident round of workgroups (4 per CU for qk, 2 for pv); each wavefront
  // then streams its blocks through the load pipeline.
  int qb = 1;
  const int qb_max = kQkScoreTokens / (kBlock * p->NT) >= 1 ? kQkScoreTokens / (kBlock * p->NT) : 1;
  while (qb < qb_max && blocks > (int64_t)kWaves * qb * 1024) qb *= 2;
  int pb = 4;  // multiple of the 4-block pv stage
  while (pb < 32 && blocks > (int64_t)kWaves * pb * 512) pb *= 2;
#ifdef SDV_TUNE_QK_BPW  // tuning builds only: fixed blocks per wavefront
  qb = min(SDV_TUNE_QK_BPW, qb_max);
#endif
#ifdef SDV_TUNE_PV_BPW
  pb = (SDV_TUNE_PV_BPW + 3) / 4 * 4;
#endif
  p->qk_bpw = qb;
  p->qk_chunk_tokens = kWaves * qb * kBlock;
  p->n_qk_chunks = (max_seq_len + p->qk_chunk_tokens - 1) / p->qk_chunk_tokens;
  p->pv_bpw = pb;
  p->pv_chunk_tokens = kWaves * pb * kBlock;
  p->n_pv_chunks = (max_seq_len + p->pv_chunk_tokens - 1) / p->pv_chunk_tokens;
  p->score_stride = max(p->n_qk_chunks * p->qk_chunk_tokens, p->n_pv_chunks * p->pv_chunk_tokens);
  const int64_t groups = (int64_t)L * B * KV;
  const size_t scores = round_up((size_t)(groups * R * p->score_stride * 2), 256);
  const size_t stats = round_up((size_t)(groups * p->n_qk_chunks * p->rpad * 8), 256);
  const size_t partial = round_up((size_t)(groups * p->n_pv_chunks * R * D * 4), 256);
  p->off_stats = scores;
  p->off_partial = scores + stats;
  p->total = scores + stats + partial;
  return true;
}

template <int D, int NT>
static void launch_qk_pv(const AttnArgs& a, const Plan& p, int zdim, hipStream_t st, int phases) {
  const unsigned gy = a.KV * p.n_row_groups;
  if (phases & SDV_PHASE_QK)
    hipLaunchKernelGGL((qk_kernel<D, NT>), dim3(p.n_qk_chunks, gy, zdim), dim3(256), 0, st, a);
  if (phases & SDV_PHASE_PV)
    hipLaunchKernelGGL((pv_kernel<D, NT>), dim3(p.n_pv_chunks, gy, zdim), dim3(256), 0, st, a);
}

template <int D>
static void launch_all(const AttnArgs& a, const Plan& p, int zdim, hipStream_t st, int phases) {
  switch (p.NT) {
    case 1: launch_qk_pv<D, 1>(a, p, zdim, st, phases); break;
    case 2: launch_qk_pv<D, 2>(a, p, zdim, st, phases); break;
    case 3: launch_qk_pv<D, 3>(a, p, zdim, st, phases); break;
    default: launch_qk_pv<D, 4>(a, p, zdim, st, phases); break;
  }
  if (phases & SDV_PHASE_REDUCE)
    hipLaunchKernelGGL(reduce_kernel<D>, dim3((a.R * D + 63) / 64, a.KV, zdim), dim3(256), 0, st, a);
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
  a.qk_bpw = p.qk_bpw;
  a.qk_chunk_tokens = p.qk_chunk_tokens;
  a.n_qk_chunks = p.n_qk_chunks;
  a.pv_bpw = p.pv_bpw;
  a.pv_chunk_tokens = p.pv_chunk_tokens;
  a.n_pv_chunks = p.n_pv_chunks;
  a.score_stride = p.score_stride;
  // RN(1/sqrt(D)): 1/sqrt(128) = 0.08838834764831845, 1/sqrt(64) = 0.125 exactly
  a.inv_sqrt_d = head_dim == 128 ? 0.08838834764831845f : 0.125f;

  hipStream_t st = static_cast<hipStream_t>(stream);
  const int zdim = num_layers * batch;
  if (head_dim == 128)
    launch_all<128>(a, p, zdim, st, phase_mask);
  else
    launch_all<64>(a, p, zdim, st, phase_mask);
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

// Kernels 2/3: paged GQA attention over BF16 K and FP8-E4M3 V, decode (q_len = 1) and
// speculative verify (q_len = k+1), with the eager path's rounding points.
//
// The reference computes (specdec/engine/model_self.py:739-776):
//   scores = bf16( bf16(q @ k^T) / sqrt(D) )        -- two BF16 roundings
//   p      = bf16( softmax_fp32(masked scores) )    -- normalised by the GLOBAL max and sum
//   out    = bf16( p @ v_hat ),  v_hat = bf16(fp32(code) * scale)   (model_self.py:316-320)
// Because p is rounded to BF16 after the global normalisation, a one-pass rescaled
// online softmax cannot reproduce it: every path takes the row statistics (max, sum) over the
// whole sequence before it forms p.  The planner (make_plan, launch_all) picks one of:
//   fused_kernel  one launch for the whole call: items of page blocks per (layer, sequence, KV
//                 head) group, statistics and partials exchanged between workgroups through
//                 the workspace's synchronisation area (also once per layer of a call too
//                 large for one launch);
//   group_kernel  256 or more one-tile groups the single launch cannot hold: persistent
//                 workgroups that each compute whole groups;
//   prefill_kernel many query rows (prefill chunks), two passes;
// and the three launches, for the rest and for the profiling split (phase_mask):
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
#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>

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
  unsigned* sync;   // fused path: expired-wait count, published statistics and partials (zero between calls)
  // fused: blocks per group, items per group, LDS width in blocks; f_layers > 0: items sized
  // per sequence (a batch with per-sequence lengths, f_layers layers)
  int f_gb, f_base, f_layers, f_maxblk;
  int64_t q_ls, q_sb, q_sh, q_ss;  // element strides of q/out: layer, batch, head, row
  int max_blocks, num_blocks, max_seq_len;
  int B, KV, S, G, R;
  int n_row_groups, rpad;
  int qk_bpw, qk_chunk_tokens, n_qk_chunks;
  int pv_bpw, pv_chunk_tokens, n_pv_chunks;
  int score_stride;
  float inv_sqrt_d;
  // in-kernel append (sdv_paged_attention_append, single launch): the S new tokens of every
  // sequence, BF16 [L][B*S][KV][D] (layers app_ls elements apart), token b*S + i at position
  // seq_len - S + i; app_v == nullptr: no append
  const uint16_t* app_k;
  const uint16_t* app_v;
  const int32_t* app_slots;
  int64_t app_ls;
  int app_scale_mode;
  // single launch: the call's tag (never 0; bit 31 set for a call recorded into a graph, whose
  // replays reuse it) and the bound of every cross-workgroup wait, in polls
  uint32_t tag;
  uint32_t spin_limit;
  // prefill pass 2: key parts per row group (1: each workgroup writes its rows' outputs itself)
  int pf_parts;
  // prefill pass 1: key parts per row group (the (max, sum) of each, per row, in stats)
  int pf_split;
  // prefill pass 2 with parts per row group by its key count (pf_kstar > 0, S a multiple of
  // the pass's rows per workgroup): at most pf_kstar blocks per part, pf_wh workgroups per
  // head; pf_parts is then the most parts of any row group (its slots per row group)
  int pf_kstar, pf_wh;
  // prefill: V dequantized once per call by pass 1 for pass 2.  Per (layer, sequence, KV head)
  // group, vh_stages stages of two page blocks, each D/16 dimension tiles x 64 lanes x 16 bytes
  // in the lane order of the p.V MFMA's A operand (lane (g, n): dimension dt*16 + n, tokens
  // 4g..4g+3 of the first block, then of the second)
  uint4* vhat;
  int vh_stages;
};

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ bf16x8 zero_bf16x8() { return __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0)); }

// max of three fp32 values in one instruction (v_max3_f32).  fmaxf on values the compiler
// cannot prove canonical (scores unpacked from BF16 bit patterns) costs a canonicalising
// v_max per operand first; the scores here are never signalling NaNs, so the plain instruction
// gives fmaxf's result.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ int seq_len_of(const AttnArgs& a, int b) {
  return a.seq_lens ? min(max(a.seq_lens[b], 0), a.max_seq_len) : a.max_seq_len;
}

// exp(x) as 2^(x * log2 e) on v_exp_f32.  The rounding of x * log2 e costs at most
// |x| * 2^-24 relative, far below one BF16 step of the probabilities it feeds (and below
// the fp32 summation noise of L); exp(-inf) = 0.
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ void merge_fast(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  const float a = (m == -INFINITY) ? 0.0f : l * fast_exp(m - mn);
  const float b = (m2 == -INFINITY) ? 0.0f : l2 * fast_exp(m2 - mn);
  m = mn;
  l = a + b;
}
// Merges of (max, sum) across lanes without LDS.  merge_fast is symmetric in its two operands
// (max, two products, one sum: no contraction across the selects), so both lanes of a pair
// get identical bits.
// merge with the lane X apart, X = 16 or 32: every lane gets merge(lower lane, upper lane)
template <int X>
__device__ __forceinline__ void merge_lanes(float& m, float& l) {
  const float2 mm = lane_pair<X>(m), ll = lane_pair<X>(l);
  m = mm.x;
  l = ll.x;
  merge_fast(m, l, mm.y, ll.y);
}
// merge with lane (lane ^ X), X = 1, 2, 4, 8: valid for the lanes lane_xor_low<X> serves
template <int X>
__device__ __forceinline__ void merge_xor_low(float& m, float& l) {
  merge_fast(m, l, lane_xor_low<X>(m), lane_xor_low<X>(l));
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
        // bf16(bf16(q.k) / sqrt(D)): for BF16 inputs, dividing by RN(sqrt(D)) and multiplying
        // by RN(1/sqrt(D)) round to the same BF16 (checked for all inputs).
        float y[4];
        round_scaled4(acc[nt][0], acc[nt][1], acc[nt][2], acc[nt][3], a.inv_sqrt_d, y);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tb + i;
          const float x = y[i];
          const bool vis = blk_ok && t < T && t <= T - a.S + qsi[nt];
          s4[i] = vis ? x : -INFINITY;
          mt = fmaxf(mt, s4[i]);
        }
        // staged in LDS: global stores mixed with the in-flight K loads would force full waits
        lsc[wave][nt * 16 + n][(j0 + u) * 4 + g] =
            make_uint2(pack_bf16x2(s4[0], s4[1]), pack_bf16x2(s4[2], s4[3]));
        if (mt != -INFINITY) {
          // exp(x - mn) as 2^(x log2 e - mn log2 e): one FMA per exp; the running sum's rescale
          // as 2^((m_old - mn) log2 e), exactly 1 while the max stays
          const float mn = fmaxf(m_run[nt], mt), nml = -mn * kLog2e;
          float l = (m_run[nt] == -INFINITY) ? 0.0f : l_run[nt] * __builtin_amdgcn_exp2f((m_run[nt] - mn) * kLog2e);
#pragma unroll
          for (int i = 0; i < 4; ++i) l += __builtin_amdgcn_exp2f(__builtin_fmaf(s4[i], kLog2e, nml));
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
  // The loop has one exit, at its head, and every path into the head has exactly one stage
  // pending (a break between the two halves would merge the other buffer's pending loads
  // into the head and make the compiler wait there); the last one or two stages are peeled
  // after it, so no stage past the wavefront's blocks is loaded (the barrier below would
  // wait for it).  The second block of a half-full last stage reads block 0 and is masked.
  const int nstg = (nb + P - 1) / P;
  if (nstg > 0) load_stage(0, ka, pa);
  int sg = 0;
  for (; sg + 2 < nstg; sg += 2) {
    load_stage((sg + 1) * P, kb, pbb);
    compute_stage(ka, pa, sg * P);
    load_stage((sg + 2) * P, ka, pa);
    compute_stage(kb, pbb, (sg + 1) * P);
  }
  if (sg + 1 < nstg) {
    load_stage((sg + 1) * P, kb, pbb);
    compute_stage(ka, pa, sg * P);
    compute_stage(kb, pbb, (sg + 1) * P);
  } else if (sg < nstg) {
    compute_stage(ka, pa, sg * P);
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float m = m_run[nt], l = l_run[nt];
    merge_lanes<16>(m, l);
    merge_lanes<32>(m, l);
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
// tile; the V page is dimension-major), the scale of token n of the block, and the 16 BF16
// scores of its query row n.  The MFMA k-slots of lane group g are tokens 8h..8h+7 of block
// g, for the two token halves h.
template <int D, int NT>
struct PvStage {
  uint4 code[D / 16];  // E4M3FN codes, token i of the block in byte i
  float scl;           // scale of token n of block g (the row broadcast hands it to the lane group)
  uint4 sc[NT][2];     // BF16 scores, tokens 0..7 and 8..15
  int blk;             // block index within the sequence (this lane group's)
  bool ok;             // the block exists and its page id is valid
};

// value of lane I of this lane's 16-lane row (DPP row_newbcast)
template <int I>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + I, 0xF, 0xF, false));
}

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
  st.scl = __builtin_nontemporal_load(slayer + page * kBlock + n);
  // scores of a block past the chunk stay inside the workspace row (score_stride covers it)
  const int64_t tok = (int64_t)min(st.blk, a.score_stride / kBlock - 1) * kBlock;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const uint4* ps = reinterpret_cast<const uint4*>(srow0 + srow_off[nt] + tok);
    st.sc[nt][0] = ps[0];
    st.sc[nt][1] = ps[1];
  }
}

// One token half (tokens 8H..8H+7 of each lane group's block) of a stage on the MFMA.
template <int D, int NT, int H>
__device__ __forceinline__ void pv_half(const PvStage<D, NT>& st, f32x4 (&acc)[D / 16][NT], const float (&gm)[NT],
                                        const float (&ginv)[NT]) {
  constexpr int DT = D / 16;
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  // P^T operand (B): probabilities of this lane's row for tokens 8H..8H+7 of its block.
  bf16x8 pop[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const uint4 w4 = st.sc[nt][H];
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
  // per-token scales of tokens 8H..8H+7 of this lane group's block
  const float s0 = row_bcast<8 * H + 0>(st.scl), s1 = row_bcast<8 * H + 1>(st.scl);
  const float s2 = row_bcast<8 * H + 2>(st.scl), s3 = row_bcast<8 * H + 3>(st.scl);
  const float s4 = row_bcast<8 * H + 4>(st.scl), s5 = row_bcast<8 * H + 5>(st.scl);
  const float s6 = row_bcast<8 * H + 6>(st.scl), s7 = row_bcast<8 * H + 7>(st.scl);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    // V_hat^T operand (A): dimension dt*16+n, tokens 8H..8H+7 of this lane group's block,
    // each bf16(f32(code) * scale) as dequantize_kv_fp8 rounds it.
    const uint32_t lo = H ? st.code[dt].z : st.code[dt].x;
    const uint32_t hi = H ? st.code[dt].w : st.code[dt].y;
    const f32x2 f01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
    const f32x2 f23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f32x2 f45 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
    const f32x2 f67 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    const bf16x8 vop = __builtin_bit_cast(
        bf16x8, make_uint4(pack_bf16x2(f01.x * s0, f01.y * s1), pack_bf16x2(f23.x * s2, f23.y * s3),
                           pack_bf16x2(f45.x * s4, f45.y * s5), pack_bf16x2(f67.x * s6, f67.y * s7)));
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[nt], acc[dt][nt], 0, 0, 0);
  }
}

template <int D, int NT>
__device__ __forceinline__ void pv_compute(PvStage<D, NT>& st, f32x4 (&acc)[D / 16][NT], const float (&gm)[NT],
                                           const float (&ginv)[NT], int T, bool stage_full, int n) {
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
    st.scl = n < nvalid ? st.scl : 0.0f;
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
  pv_half<D, NT, 0>(st, acc, gm, ginv);
  pv_half<D, NT, 1>(st, acc, gm, ginv);
}

template <int D, int NT>
__global__ __launch_bounds__(256) void pv_kernel(AttnArgs a) {
  constexpr int DT = D / 16;  // 16-dimension MFMA tiles
  constexpr int RT = NT * 16;
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

  // Chunk statistics of this lane's query rows, issued before the V loads so that waiting
  // for them leaves V in flight.  Lane group g merges chunks g, g+4, ... in order.
  const int nvq = (T + a.qk_chunk_tokens - 1) / a.qk_chunk_tokens;
  float sm[NT], sl[NT];
  {
    const float2* st0 = a.stats + (int64_t)grp * a.n_qk_chunks * a.rpad;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int rr = rg * RT + nt * 16 + n;
      const float2* st = st0 + (rr < a.R ? rr : 0);
      float m = -INFINITY, l = 0.0f;
      int cc = g;
      for (; cc + 12 < nvq; cc += 16) {
        float2 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = st[(int64_t)(cc + 4 * u) * a.rpad];
#pragma unroll
        for (int u = 0; u < 4; ++u) merge_fast(m, l, v[u].x, v[u].y);
      }
      for (; cc < nvq; cc += 4) {
        const float2 v = st[(int64_t)cc * a.rpad];
        merge_fast(m, l, v.x, v.y);
      }
      sm[nt] = m;
      sl[nt] = l;
    }
  }
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

  // Stages 0 and 1 of V are in flight while the statistics are merged.  These two loads are
  // unconditional (a stage past the end reads block 0 and is never computed), so the wait
  // for the statistics, issued before them, does not wait for them.
  const int nst = (nb + 3) >> 2;
  PvStage<D, NT> sa, sb;
  pv_load<D, NT>(sa, a, 0, my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);
  pv_load<D, NT>(sb, a, 4, my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);

  // global (M, 1/L) of each row: the four lane groups' partial merges combine in a fixed
  // tree (xor 16, then xor 32), so every lane, wave and workgroup gets identical values.
  float gm[NT], ginv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float m = sm[nt], l = sl[nt];
    merge_lanes<16>(m, l);
    merge_lanes<32>(m, l);
    gm[nt] = m;
    ginv[nt] = 1.0f / l;
  }

  f32x4 acc[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[dt][nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // Ping-pong over stages.  A stage is "full" (no masking) when all 64 of its slots are
  // tokens of the sequence -- wave-uniform.
  const int full_stages = min(nb, max(0, (T >> 4) - blk0)) >> 2;
  // Full rounds (both reloads stages of the wavefront) in the loop, the last one to three
  // stages after it: no stage past the end is loaded there (the barrier below would wait
  // for it).
  int st_i = 0;
  for (; st_i + 3 < nst; st_i += 2) {
    pv_compute<D, NT>(sa, acc, gm, ginv, T, st_i < full_stages, n);
    pv_load<D, NT>(sa, a, 4 * (st_i + 2), my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);
    pv_compute<D, NT>(sb, acc, gm, ginv, T, st_i + 1 < full_stages, n);
    pv_load<D, NT>(sb, a, 4 * (st_i + 3), my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);
  }
  if (st_i < nst) {
    pv_compute<D, NT>(sa, acc, gm, ginv, T, st_i < full_stages, n);
    if (st_i + 2 < nst) pv_load<D, NT>(sa, a, 4 * (st_i + 2), my_pb, nb, blk0, vlayer, slayer, srow0, srow_off, kvh, g, n);
  }
  if (st_i + 1 < nst) pv_compute<D, NT>(sb, acc, gm, ginv, T, st_i + 1 < full_stages, n);
  if (st_i + 2 < nst) pv_compute<D, NT>(sa, acc, gm, ginv, T, st_i + 2 < full_stages, n);

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

// ---------------------------------------------------------------------------- in-kernel append
// The new tokens of one (layer, sequence, KV head) whose positions fall in page blocks
// [blk_lo, blk_hi) of the sequence, written into the pages exactly as sdv_quant_append writes
// them (scale per token and KV head, E4M3FN codes, BF16 K copy; the same helpers): wavefront w
// takes positions w, w + W, ...; lanes p < D/8 hold dimensions 8p .. 8p+7 of the token.
template <int D, int W>
__device__ __forceinline__ void append_new_tokens(const AttnArgs& a, int layer, int b, int kvh, int T, int blk_lo,
                                                  int blk_hi, int wave, int lane) {
  constexpr int LPR = D / 8;
  const int first = T - a.S;  // position of new token 0
  const int p_lo = max(max(first, blk_lo * kBlock), 0), p_hi = min(T, blk_hi * kBlock);
  const int64_t n_slots = (int64_t)a.num_blocks * kBlock;
  const int p = lane < LPR ? lane : 0;
  uint16_t* kp = const_cast<uint16_t*>(a.k_pages) + layer * a.k_ls;
  uint8_t* vp = const_cast<uint8_t*>(a.v_pages) + layer * a.v_ls;
  float* sp = const_cast<float*>(a.v_scales) + layer * a.s_ls;
  for (int pos = p_lo + wave; pos < p_hi; pos += W) {  // wave-uniform
    const int row = b * a.S + (pos - first);
    const int slot = a.app_slots ? a.app_slots[row]
                                 : table_slot(a.block_table + (int64_t)b * a.max_blocks, a.max_blocks, a.num_blocks, pos);
    if (slot < 0 || (int64_t)slot >= n_slots) continue;
    const int64_t in = layer * a.app_ls + ((int64_t)row * a.KV + kvh) * D + 8 * p;
    const uint4 vw = *reinterpret_cast<const uint4*>(a.app_v + in);
    const uint4 kw = *reinterpret_cast<const uint4*>(a.app_k + in);
    float sc, rcp;
    bool fast;
    token_scale(row_max_bits<LPR>(abs_max_bits8(vw)), a.app_scale_mode, sc, rcp, fast);
    const int blk = slot >> 4, off = slot & (kBlock - 1);
    const int64_t page = (int64_t)blk * a.KV + kvh;
    if (lane < LPR) {
      const uint32_t w[4] = {vw.x, vw.y, vw.z, vw.w};
      uint8_t* vrow = vp + (page * D + 8 * p) * kBlock + off;
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        const float x0 = __uint_as_float(w[k >> 1] << 16), x1 = __uint_as_float(w[k >> 1] & 0xFFFF0000u);
        uint32_t c2;
        if (fast) {
          c2 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(quotient_rn(x0, sc, rcp), quotient_rn(x1, sc, rcp), 0,
                                                          false);
        } else {  // max-abs not finite or in (0, 2^-60): exact division and the integer encoder
          c2 = e4m3fn_encode(x0 / sc) | (e4m3fn_encode(x1 / sc) << 8);
        }
        vrow[k * kBlock] = (uint8_t)c2;
        vrow[(k + 1) * kBlock] = (uint8_t)(c2 >> 8);
      }
      *reinterpret_cast<uint4*>(kp + page * kBlock * D + (p * kBlock + off) * 8) = kw;
      if (lane == 0) sp[page * kBlock + off] = sc;
    }
  }
}

// ---------------------------------------------------------------------------- fused
// One launch for the shapes whose whole grid fits the device at once (one query-row group:
// decode and verify).  One workgroup per CU (W = 8 wavefronts for one or two row tiles, 4 when
// the row tiles need more registers), each owning one item: a run of page blocks of one
// (layer*batch, KV head) group.  Every group is cut into the same number of items of nearly
// equal size, so every busy CU streams the same number of bytes (a batch with per-sequence
// lengths sizes each sequence's items from its length instead: f_layers, below).  Inside a
// workgroup wavefront w takes blocks (and p.V units) w, w + W, ...: a fixed trip count lets
// each streaming loop end without loads past its last block.  Per workgroup:
//   1. q.k^T over the item's blocks: BF16 scores and per-block (max, sum) of every row into
//      LDS; the item's (max, sum) -- merged over its blocks in block order, so it does not
//      depend on which wavefront took which block -- published to device memory as words
//      tagged with the call (below): no counter is needed for this step.
//   2. Once every item of the group has published (one wavefront polls, the others keep
//      their first V loads in flight), the group's statistics are merged in a
//      fixed order; the item's scores in LDS become p = bf16(exp(s - M) / L) in place, once
//      per (row, token); the wavefronts run p.V over the item's blocks, each summing its
//      units in registers; the wavefronts' sums are added in LDS in wavefront order and the
//      fp32 partial is published.
//   3. Workgroup c of the group owns a slice of the outputs: it polls the slice of every
//      item's partial, sums it over the items in order (the result does not depend on the
//      order workgroups finish) into the BF16 output, and clears a share of the statistics
//      for the next call (partial slots are zeroed by their own item at the next call's start).
// Cross-workgroup data moves through device-scope (sc1) stores and loads, which bypass the
// per-XCD L2 caches; no counter, ticket or cache-writeback fence is needed (on gfx950 each
// agent-scope release costs ~40 ns and serialises chip-wide; a counter round trip costs ~1.3 us
// across XCDs).  A word left over from an earlier call never passes for a current one:
//   * statistics travel as 64-bit (value, call tag) words written and read with
//     single-copy-atomic 64-bit accesses; a reader takes a word only when it carries its own
//     call's tag.  Eager calls get a fresh tag each; the replays of a graph reuse their recorded
//     tag, so the owners clear the statistics they consumed and every replay starts clean.
//   * a partial word holds the float's bits + 1 (0 means "not yet written").  An item zeroes
//     its own partial slot at the start of the call and waits for those stores to complete
//     before it publishes its statistics; an owner reads partials only after it has taken every
//     item's statistics of this call, so whatever it reads in a slot was written by that item in
//     this call.
// Deadlock freedom: a workgroup publishes before it waits and the grid never exceeds the
// device's resident capacity (occupancy query), so every entry a wait needs comes from a
// running workgroup.  If that assumption fails (another process holds CUs, a CU mask), waits
// are bounded (a.spin_limit polls): an expired wait counts in word 0 of the synchronisation
// area, turns the affected outputs into NaN (its group's statistics, or the owner's output
// slice) and skips the clears.  A graph-recorded call that expires also sets word 1: from
// then on every graph-recorded call writes NaN to all of its outputs and counts itself
// instead of running (its replays would reuse the tag of the words that may be left over)
// until sdv_attention_workspace_init clears the area; eager calls are unaffected.
constexpr int kFusedMaxItems = 4096;    // published (max, sum) rows: 64 per item
constexpr int kFusedMaxChunks = 64;     // items per group
// Most items per group.  A one-layer call is split as finely as this allows; 32 items (4
// blocks each at T=2048, 16 at 8K) beat 64 (10.2-10.5 vs 10.9 us at 2K; 28 per-layer calls in
// a graph 13.0 vs 13.4 us per layer at 8K): fewer entries to merge and sum per group.
constexpr int kFusedGroupItems = 32;
static_assert(kFusedGroupItems <= kFusedMaxChunks, "the output stage holds kFusedMaxChunks items");
// Resident workgroups per CU the planner allows (the occupancy query may allow more).  Decode
// (one row tile) keeps one workgroup per CU: a second resident workgroup only splits the CU's
// bandwidth between two items of the same size (28 layers at 8K: 504 workgroups 42.7-43.1 us
// against 224 at 39.4 us).  The D=128 verify shapes keep the counts they were tuned at (one for
// two row tiles, two for three or four).
template <int D, int NT>
constexpr int fused_max_per_cu() { return NT == 1 ? 1 : D == 128 ? (NT == 2 ? 1 : 2) : 64; }
constexpr size_t kSyncHeadBytes = 256;  // word 0: expired waits and refused calls; word 1: graph poison
constexpr size_t kSyncStatsBytes = (size_t)kFusedMaxItems * 64 * 16;  // (max, tag), (sum, tag) per row
constexpr size_t kSyncPartBytes = (size_t)8 << 20;  // fp32 partials (bits + 1) of one call's items
constexpr size_t kSyncBytes = kSyncHeadBytes + kSyncStatsBytes + kSyncPartBytes;
static_assert(kSyncBytes == SDV_SYNC_BYTES, "sdv.h states the synchronisation prefix size");
constexpr uint32_t kTagGraph = 0x80000000u;  // tag bit of a graph-recorded call
constexpr uint32_t kDefaultSpinLimit = 1u << 20;

// Phase timeline of the single launch, in builds with SDV_PHASE_TRACE only (libsdv_trace.so):
// thread 0 of each of the first kPhaseTraceGroups workgroups stamps the 100 MHz wall clock at
// the phase boundaries 0..9 (start, table + append done, q.k^T done, statistics published,
// group statistics read, p.V done, partial published, owner polls and output sums done,
// output written, end)
// of fused_kernel into LDS and writes its kPhaseSlots words out at the end (a global store per
// stamp would make the next barrier wait for it: __syncthreads waits for the wavefront's
// outstanding stores); sdv_phase_trace_read copies the array to the host.  The product library
// compiles the stamps away.
constexpr int kPhaseSlots = 16;
constexpr int kPhaseTraceGroups = 4096;
#ifdef SDV_PHASE_TRACE
__device__ unsigned long long phase_trace[kPhaseTraceGroups * kPhaseSlots];
#define SDV_PHASE_DECL                                                                      \
  __shared__ unsigned long long s_phase[kPhaseSlots];                                       \
  if (threadIdx.x == 0)                                                                     \
    for (int i_ = 0; i_ < kPhaseSlots; ++i_) s_phase[i_] = 0
#define SDV_PHASE(k)                                                                        \
  do {                                                                                      \
    if (threadIdx.x == 0) s_phase[(k)] = wall_clock64();                                    \
  } while (0)
#define SDV_PHASE_FLUSH()                                                                   \
  do {                                                                                      \
    if (threadIdx.x == 0 && blockIdx.x < kPhaseTraceGroups)                                 \
      for (int i_ = 0; i_ < kPhaseSlots; ++i_) phase_trace[blockIdx.x * kPhaseSlots + i_] = s_phase[i_]; \
  } while (0)
// group_kernel accumulates per workgroup: words 10-12 = wall-clock ticks in claim + setup, q.k^T
// (with the statistics merge) and p.V (with the output); word 13 = groups done.
#define SDV_PHASE_ADD(k, v)                                                                 \
  do {                                                                                      \
    if (threadIdx.x == 0 && blockIdx.x < kPhaseTraceGroups)                                 \
      phase_trace[blockIdx.x * kPhaseSlots + (k)] += (v);                                   \
  } while (0)
#define SDV_CLOCK() wall_clock64()
#else
#define SDV_PHASE_DECL \
  do {                 \
  } while (0)
#define SDV_PHASE(k) \
  do {               \
  } while (0)
#define SDV_PHASE_FLUSH() \
  do {                    \
  } while (0)
#define SDV_PHASE_ADD(k, v) \
  do {                      \
  } while (0)
#define SDV_CLOCK() 0ull
#endif

__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag) {
  return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)tag << 32);
}
__device__ __forceinline__ void store_dev_u64(uint64_t* p, uint64_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool has_tag(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float word_value(uint64_t w) { return __builtin_bit_cast(float, (uint32_t)w); }
// statistics of (item, row): words 2*(item*64 + row) (max) and +1 (sum)
__device__ __forceinline__ uint64_t* sync_stats(const AttnArgs& a) {
  return reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(a.sync) + kSyncHeadBytes);
}
// partial of (item, output element o): float item * R * D + o
__device__ __forceinline__ float* sync_parts(const AttnArgs& a) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(a.sync) + kSyncHeadBytes + kSyncStatsBytes);
}
__device__ __forceinline__ void count_sync_error(const AttnArgs& a) {
  __hip_atomic_fetch_add(a.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A published partial word holds the float's bits + 1, so 0 always means "not yet written"
// (the one pattern that would wrap, NaN 0xFFFFFFFF, is stored as a quiet NaN).
__device__ __forceinline__ uint32_t part_word(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return u == 0xFFFFFFFFu ? 0x7FC00001u : u + 1u;
}
__device__ __forceinline__ u32x4_t part_enc(f32x4 v) {
  return (u32x4_t){part_word(v[0]), part_word(v[1]), part_word(v[2]), part_word(v[3])};
}
__device__ __forceinline__ float4 part_dec(u32x4_t w) {
  return make_float4(__builtin_bit_cast(float, w[0] - 1u), __builtin_bit_cast(float, w[1] - 1u),
                     __builtin_bit_cast(float, w[2] - 1u), __builtin_bit_cast(float, w[3] - 1u));
}
#define SDV_VMCNT0() __builtin_amdgcn_s_waitcnt(0x0F70)  // vmcnt(0); exp/lgkm counters untouched

// wavefronts of the fused workgroup for NT row tiles.  With one row tile the workgroup is
// alone on its CU; measured on gfx950, 8 wavefronts finish a D=128 call sooner than 16 (one
// layer at T=2048: 12.6 us vs 13.7 us; 28 layers at 8K: equal within noise), and since the
// streaming loops stopped loading past their items also a D=64 call (24 layers at 8K:
// 21.8 -> 21.5 us, at 2K 13.05 -> 12.5 us; one layer at 2K 8.97 -> 8.49 us; with the
// counter-claimed loops 16 had been faster for D=64: 23.7 us against 25.5 us at 8K).
template <int D, int NT>
constexpr int fused_waves() { return NT <= 2 ? 8 : 4; }
constexpr int kVStages = 6;  // p.V stages in flight per wavefront (one 16-dimension tile each)
// dimension-tile groups of the static p.V split (several row tiles): wavefront w takes the
// 16-dimension tiles of group w % ntg for block part w / ntg
__host__ __device__ constexpr int fused_ntg(int D, int W) { return D / 16 < W ? D / 16 : W; }
// Two row tiles with items of at least kWideMinBlocks blocks: two groups of wider tiles
// (D/32 dimensions per wavefront over a quarter of the blocks).  The conversion of the codes,
// the scale broadcasts, the address arithmetic and the probability reads are then shared by
// four tiles instead of one; the verify p.V is bound by that VALU work (per-wavefront end
// times on 28 layers at 8K: the second wavefront of every SIMD ends 2.4 us after the first).
// Small items keep one tile per wavefront: with a few blocks per part the parts' sum costs
// more than it saves (28 layers, S=5: 8K 49.6-51.9 -> 48.4-48.9 us; 2K and 4K equal within
// noise; one layer 1.1 us slower at 8K with 16 blocks per item).
constexpr int kWideMinBlocks = 64;
__host__ __device__ constexpr int fused_ntg_wide(int D, int W, int NT) {
  return NT == 2 && fused_ntg(D, W) > 2 ? 2 : fused_ntg(D, W);
}

// dynamic LDS of a fused workgroup with items of up to `maxblk` blocks (byte offsets).  With
// one row tile the p.V work is split in units and each unit's result gets an LDS slot
// ([stage][R][D] floats); otherwise the parts of the static split ([parts][R][D]).
struct FusedLds {
  int scores, bstats, pages, gstats, parts, total;
};
__host__ __device__ inline FusedLds fused_lds_layout(int R, int D, int maxblk, int W, bool unit_pv, int ntg) {
  const int tp = W / ntg;
  FusedLds l;
  l.scores = 0;                                                            // [R][16*maxblk + 8] bf16
  l.bstats = (l.scores + R * (maxblk * kBlock + 8) * 2 + 15) & ~15;        // [maxblk][R] float2
  l.pages = l.bstats + maxblk * R * 8;                                     // [maxblk] int
  l.gstats = (l.pages + maxblk * 4 + 15) & ~15;                           // [64] float2
  if (unit_pv) {  // one slot of R rows x (up to) 64 dimensions per wavefront
    l.parts = l.gstats + 64 * 8;
    l.total = l.parts + W * R * (D < 64 ? D : 64) * 4;
  } else {
    // the static split's parts are written after every wavefront has finished p.V: they
    // reuse the scores from offset 0
    l.parts = 0;
    l.total = l.gstats + 64 * 8;
    const int parts_bytes = (tp > 1 ? tp : 0) * R * D * 4;
    if (l.total < parts_bytes) l.total = parts_bytes;
  }
  return l;
}

template <int D, int NT, int W, int NTG>
__global__ __launch_bounds__(64 * W) void fused_kernel(AttnArgs a) {
  constexpr int NTHR = 64 * W;
  constexpr int KK = D / 32, DT = D / 16;
  // NTG: dimension-tile groups in p.V (static split)
  constexpr int DTW = DT / NTG;          // 16-dimension tiles per wavefront
  constexpr int TP = W / NTG;            // block parts in p.V
  constexpr int P = 1;                   // page blocks per q.k^T stage
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  extern __shared__ uint4 smem_u4[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int item = blockIdx.x;
  SDV_PHASE_DECL;
  SDV_PHASE(0);
  {
    // one field of each 64-byte line of the arguments, loaded together: the compiler fetches
    // the arguments where they are first used, and each first touch of a line is a
    // scalar-cache miss that the prologue would wait for in turn (one layer at 8K: 11.56 ->
    // 11.08 us; the empty asm only makes the values live here)
    const uint64_t l0 = (uint64_t)a.q;
    const int l1 = a.f_base, l2 = a.max_seq_len;
    const float l3 = a.inv_sqrt_d;
    const uint32_t l4 = a.tag;
    asm volatile("" ::"s"(l0), "s"(l1), "s"(l2), "s"(l3), "s"(l4));
  }
  int grp, c, n_g, item0, gbg;  // group, item in it, its items, its first item, its blocks
  if (a.f_layers > 0) {
    // A batch with per-sequence lengths (at most 64 sequences, one per lane): the groups of
    // sequence b get ceil(blocks_b / S) items -- at most kFusedGroupItems, at most one per
    // block, one for an empty sequence -- with S the smallest item size whose items fit the
    // grid, found by bisection over [1, f_maxblk] (S = f_maxblk fits: the host plan gives every
    // group f_base items of at most f_maxblk blocks).  Long sequences are cut finer than short
    // ones instead of every group getting the items of the longest, and no item exceeds
    // f_maxblk blocks (LDS).  Every workgroup derives the same plan from seq_lens; workgroups
    // past it exit.  Items of layer l, sequence b, KV head h start at
    // l * KV * sum(items) + KV * prefix_b + h * items_b.
    const int B = a.B, L = a.f_layers, gs = L * a.KV;  // groups per sequence
    const int Tb = lane < B ? seq_len_of(a, lane) : 0;
    const int blk = (Tb + kBlock - 1) >> 4;
    auto items_for = [&](int sz) {  // sz: wave-uniform item size
      return lane < B ? (Tb == 0 ? 1 : min(min(kFusedGroupItems, blk), (blk + sz - 1) / sz)) : 0;
    };
    auto wave_sum = [&](int v) {  // exact: at most 64 * 32 items
      float f = (float)v;
      f += lane_xor_low<1>(f);
      f += lane_xor_low<2>(f);
      f += lane_xor_low<4>(f);
      f += lane_xor_low<8>(f);
      float2 pr = lane_pair<16>(f);
      f = pr.x + pr.y;
      pr = lane_pair<32>(f);
      f = pr.x + pr.y;
      return (int)__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f)));  // lane 0 holds the sum
    };
    int lo = 1, hi = a.f_maxblk;
    while (lo < hi) {  // wave-uniform
      const int mid = (lo + hi) >> 1;
      if (gs * wave_sum(items_for(mid)) <= (int)gridDim.x)
        hi = mid;
      else
        lo = mid + 1;
    }
    const int items = items_for(lo);
    int incl = items;  // inclusive prefix over the sequences
    for (int off = 1; off < kWave; off <<= 1) {
      const int v = __shfl_up(incl, off);
      if (lane >= off) incl += v;
    }
    // readlane: the plan's values are wave-uniform and stay scalar (as __shfl results they
    // made the item arithmetic after this point vector code: +24 VGPRs, verify 3 us slower)
    const int per_layer = a.KV * __builtin_amdgcn_readlane(incl, kWave - 1);
    const int li = item / per_layer;
    if (li >= L) return;  // workgroup-uniform: past the plan
    const int r = item - li * per_layer;
    const int excl = incl - items;
    const uint64_t mine = __ballot(lane < B && r >= a.KV * excl && r < a.KV * incl);
    const int bs = __builtin_ctzll(mine);  // the sequence
    n_g = __builtin_amdgcn_readlane(items, bs);
    gbg = __builtin_amdgcn_readlane(blk, bs);
    const int rr = r - a.KV * __builtin_amdgcn_readlane(excl, bs);
    const int h = rr / n_g;
    c = rr - h * n_g;
    item0 = item - c;
    grp = (li * B + bs) * a.KV + h;
  } else {
    n_g = a.f_base;
    grp = item / n_g;
    c = item - grp * n_g;
    item0 = grp * n_g;
    gbg = a.f_gb;
  }
  // 32-bit products and quotients: a group has at most 32 items and (items of at most
  // 160 KiB of LDS) fewer than 2^18 blocks, so they stay far below 2^31 (a 64-bit division
  // is a long software sequence in a prologue every call waits for)
  const int blk_lo = (int)((unsigned)(c * gbg) / (unsigned)n_g);
  const int nbk = (int)((unsigned)((c + 1) * gbg) / (unsigned)n_g) - blk_lo;  // item blocks, 1..f_maxblk
  const int zb = grp / a.KV, kvh = grp - zb * a.KV, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int tok0 = blk_lo * kBlock;
  if (tok0 >= T) {
    if (T == 0 && c == 0) {  // empty sequence: the eager sum over no keys is 0
      for (int o = tid; o < a.R * D; o += NTHR) {
        const int row = o / D, d = o - row * D, hl = row / a.S, si = row % a.S;
        a.out[layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + d] = 0;
      }
    }
    return;  // workgroup-uniform
  }
  const int nblk_seq = (T + kBlock - 1) >> 4;
  const int nbv = min(nbk, nblk_seq - blk_lo);  // item blocks inside the sequence (>= 1)
  // non-empty items of the group: item i starts at block floor(i * gb / n_g)
  const int nvq = min(n_g, (int)((unsigned)(nblk_seq * n_g + gbg - 1) / (unsigned)gbg));
  // Output slice of this workgroup: workgroup c < nvq of the group owns 16-byte output chunks
  // [lo, lo + w) (four outputs each); nown workgroups have a non-empty slice.
  const int n4 = a.R * D / 4;
  const int per = (n4 + nvq - 1) / nvq;
  const int lo = c * per, w = max(min(n4, lo + per) - lo, 0);
  const int nown = (n4 + per - 1) / per;
  // NaN into this workgroup's output slice (a failed or refused call)
  auto nan_slice = [&]() {
    for (int o = tid; o < w; o += NTHR) {
      const int o4 = lo + o;
      const int row = (4 * o4) / D, d = 4 * o4 - row * D, hl = row / a.S, si = row % a.S;
      uint16_t* dst = a.out + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + d;
      *reinterpret_cast<uint2*>(dst) = make_uint2(0x7FC07FC0u, 0x7FC07FC0u);
    }
  };
  const bool graph_call = (a.tag & kTagGraph) != 0;
  __shared__ int s_fail;  // a wait of this workgroup expired (or a graph-recorded call was refused)
  const int64_t pstride = (int64_t)a.R * D;  // floats per item
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(sync_parts(a), (short)0, (int)kSyncPartBytes, 0x00020000);

  constexpr bool kUnitPV = NT == 1;  // one row tile: p.V in units spread over the wavefronts
  const FusedLds lay = fused_lds_layout(a.R, D, a.f_maxblk, W, kUnitPV, NTG);
  char* smem = reinterpret_cast<char*>(smem_u4);
  uint16_t* lsc = reinterpret_cast<uint16_t*>(smem + lay.scores);  // row r: scores of query row r
  const int lrow = a.f_maxblk * kBlock + 8;
  float2* bst = reinterpret_cast<float2*>(smem + lay.bstats);      // [block][row] (max, sum)
  int* lpb = reinterpret_cast<int*>(smem + lay.pages);              // page ids of the item blocks
  const int* btrow = a.block_table + (int64_t)b * a.max_blocks;
  for (int j = tid; j < nbv; j += NTHR) {
    const int pb = btrow[blk_lo + j];
    lpb[j] = (pb >= 0 && pb < a.num_blocks) ? pb : -1;
  }
  if (tid == 0) s_fail = 0;
  // the group's new tokens inside this item's blocks go into the pages first; the barrier
  // (workgroup-scope release and acquire) makes them visible to the loads below, and only
  // this workgroup reads these blocks
  if (a.app_v) {
    append_new_tokens<D, W>(a, layer, b, kvh, T, blk_lo, blk_lo + nbk, wave, lane);
    __threadfence_block();
  }
  __syncthreads();

  SDV_PHASE(1);
  // ------------------------------------------------------------------ 1. q.k^T
  bf16x8 qop[NT][KK];
  int qsi[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = nt * 16 + n;
    const bool rv = row < a.R;
    const int hl = rv ? row / a.S : 0;
    qsi[nt] = rv ? row % a.S : 0;
    const uint16_t* qp =
        a.q + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + qsi[nt] * a.q_ss + g * 8;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qop[nt][kk] = rv ? load_bf16x8(qp + kk * 32) : zero_bf16x8();
  }
  {
    const uint16_t* kbase = a.k_pages + layer * a.k_ls + (int64_t)lane * 8;
    auto load_stage = [&](int j0, bf16x8 (&kop)[P][KK], int (&pbs)[P]) {
#pragma unroll
      for (int u = 0; u < P; ++u) {
        pbs[u] = (j0 + u < nbv) ? lpb[j0 + u] : -1;
        const uint16_t* kp = kbase + ((int64_t)max(pbs[u], 0) * a.KV + kvh) * (kBlock * D);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) kop[u][kk] = __builtin_bit_cast(bf16x8, load_stream16(kp + kk * 512));
      }
    };
    auto compute_stage = [&](const bf16x8 (&kop)[P][KK], const int (&pbs)[P], int j0) {
#pragma unroll
      for (int u = 0; u < P; ++u) {
        const int jb = j0 + u;  // block within the item
        if (jb >= nbv) break;
        const int tb = tok0 + jb * kBlock + 4 * g;  // this lane's first token
        const bool blk_ok = pbs[u] >= 0;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f32x4 acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[u][kk], qop[nt][kk], acc, 0, 0, 0);
          float s4[4];
          float mt = -INFINITY;
          float y[4];
          round_scaled4(acc[0], acc[1], acc[2], acc[3], a.inv_sqrt_d, y);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = tb + i;
            const float x = y[i];
            const bool vis = blk_ok && t < T && t <= T - a.S + qsi[nt];
            s4[i] = vis ? x : -INFINITY;
            mt = fmaxf(mt, s4[i]);
          }
          const int row = nt * 16 + n;
          if (row < a.R)
            *reinterpret_cast<uint2*>(lsc + row * lrow + jb * kBlock + 4 * g) =
                make_uint2(pack_bf16x2(s4[0], s4[1]), pack_bf16x2(s4[2], s4[3]));
          // this block's (max, sum) of the row: the block max over the four lane groups first,
          // then every exp against it and a fixed sum tree (lower lane first, so the lanes of
          // a pair hold identical bits).  Against a (max, sum) merge per lane-group pair this
          // spends no rescaling exps: the q.k^T phase of verify is partly VALU-bound.
          float2 pm = lane_pair<16>(mt);
          float M = fmaxf(pm.x, pm.y);
          pm = lane_pair<32>(M);
          M = fmaxf(pm.x, pm.y);
          const float nml = M == -INFINITY ? 0.0f : -M * kLog2e;  // empty row: every exp is 0
          float l = 0.0f;
#pragma unroll
          for (int i = 0; i < 4; ++i) l += __builtin_amdgcn_exp2f(__builtin_fmaf(s4[i], kLog2e, nml));
          float2 pl = lane_pair<16>(l);
          l = pl.x + pl.y;
          pl = lane_pair<32>(l);
          l = pl.x + pl.y;
          if (g == 0 && row < a.R) bst[jb * a.R + row] = make_float2(M, l);
        }
      }
    };
    // Wavefront w streams blocks w, w + W, ... (ns of them), two in flight: the loop body
    // loads the next two blocks while it multiplies the current ones, and the last one or two
    // are peeled after it, so every path into the loop head has exactly one block pending
    // (the wait before each multiply is exact) and no load goes past the item.  Claiming
    // blocks from an LDS counter instead needs a load of some block after the last claim to
    // keep the waits exact, and the barrier below then waits for that load (one layer at 8K:
    // 13.1 -> 12.8 us with the p.V units below done the same way).
    bf16x8 ka[P][KK], kb[P][KK];
    int pa[P], pbb[P];
    const int ns = wave < nbv ? (nbv - 1 - wave) / W + 1 : 0;  // blocks wave, wave + W, ...
    if (ns > 0) load_stage(wave, ka, pa);
    // This item's partial slot starts the call zeroed: the stores go out behind the first K
    // loads (a wait for those loads does not cover them) and have completed before the item
    // publishes its statistics (the barrier and vmcnt(0) after q.k^T).  Issued before the
    // block-table barrier, which waits for them, they cost one-layer calls about 0.5 us.
    for (int o4 = tid; o4 < n4; o4 += NTHR)
      __builtin_amdgcn_raw_buffer_store_b128((u32x4_t){0u, 0u, 0u, 0u}, prs, (int)((item * pstride + 4 * o4) * 4), 0, 16);
    if (ns > 0) {
      int s = 0;
      while (s + 2 < ns) {
        load_stage(wave + (s + 1) * W, kb, pbb);
        compute_stage(ka, pa, wave + s * W);
        load_stage(wave + (s + 2) * W, ka, pa);
        compute_stage(kb, pbb, wave + (s + 1) * W);
        s += 2;
      }
      if (s + 1 < ns) {
        load_stage(wave + (s + 1) * W, kb, pbb);
        compute_stage(ka, pa, wave + s * W);
        compute_stage(kb, pbb, wave + (s + 1) * W);
      } else {
        compute_stage(ka, pa, wave + s * W);
      }
    }
  }
  __syncthreads();
  // the zeroing stores of this item's partial slot have completed before its statistics are
  // published
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  SDV_VMCNT0();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  SDV_PHASE(2);
  uint64_t* fs = sync_stats(a);
  // the item's statistics of each row, in an order that does not depend on which wavefront
  // took which block in q.k^T: the row's max over the item's blocks first, then each block's
  // sum rescaled once against it and added along a fixed tree (one exp per block and no
  // branches, where a pairwise (max, sum) merge spends two exps and a branch per tree level).
  // One row per wavefront (decode): lane l takes blocks l, l+64, ... in order, then a tree
  // over the 64 lanes whose result lane 0 holds.  More rows (verify): the wavefront owns rows
  // wave, wave + W, ... (rpw of them) and gives each a group of lpr lanes, so all its rows go
  // through one pass (lane sl of a group takes blocks sl, sl + lpr, ... in order, then a tree
  // inside the group whose result the group's first lane holds).
  auto publish_stat = [&](int row, float m, float l) {
    uint64_t* p = fs + 2 * ((int64_t)item * 64 + row);
    store_dev_u64(p, tagged(m, a.tag));
    store_dev_u64(p + 1, tagged(l, a.tag));
  };
  // one block's sum rescaled to the row max M (an empty block adds 0)
  auto rescaled = [&](float2 v, float M) { return v.x == -INFINITY ? 0.0f : v.y * fast_exp(v.x - M); };
  const int rpw = (a.R + W - 1) / W;  // <= 16: R <= 64 rows, W >= 4
  if (rpw == 1) {
    if (wave < a.R) {
      // lane 0 takes lanes 1, 2, 4 and 8 (row shifts and quad permutes), then rows 16 and 32
      // apart.  Lanes >= nbv hold nothing, so the tree only spans the first nbv lanes
      // (wave-uniform tests).
      float m = -INFINITY;
      for (int j = lane; j < nbv; j += kWave) m = fmaxf(m, bst[j * a.R + wave].x);
      if (nbv > 1) m = fmaxf(m, lane_xor_low<1>(m));
      if (nbv > 2) m = fmaxf(m, lane_xor_low<2>(m));
      if (nbv > 4) m = fmaxf(m, lane_xor_low<4>(m));
      if (nbv > 8) m = fmaxf(m, lane_xor_low<8>(m));
      if (nbv > 16) { const float2 p2 = lane_pair<16>(m); m = fmaxf(p2.x, p2.y); }
      if (nbv > 32) { const float2 p2 = lane_pair<32>(m); m = fmaxf(p2.x, p2.y); }
      const float M = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(m)));  // lane 0: the row max
      float l = 0.0f;
      for (int j = lane; j < nbv; j += kWave) l += rescaled(bst[j * a.R + wave], M);
      if (nbv > 1) l += lane_xor_low<1>(l);
      if (nbv > 2) l += lane_xor_low<2>(l);
      if (nbv > 4) l += lane_xor_low<4>(l);
      if (nbv > 8) l += lane_xor_low<8>(l);
      if (nbv > 16) { const float2 p2 = lane_pair<16>(l); l = p2.x + p2.y; }
      if (nbv > 32) { const float2 p2 = lane_pair<32>(l); l = p2.x + p2.y; }
      if (lane == 0) publish_stat(wave, M, l);
    }
  } else {
    const int lpr = rpw <= 2 ? 32 : rpw <= 4 ? 16 : rpw <= 8 ? 8 : 4;
    const int sub = lane / lpr, sl = lane - sub * lpr;
    const int row = wave + W * sub;
    const bool act = sub < rpw && row < a.R;
    // the group leaders (sl = 0: lanes that are multiples of lpr) take lanes 1, 2, 4, 8 and 16
    // apart, as far as the group reaches (wave-uniform tests)
    float m = -INFINITY;
    if (act)
      for (int j = sl; j < nbv; j += lpr) m = fmaxf(m, bst[j * a.R + row].x);
    m = fmaxf(m, lane_xor_low<1>(m));
    m = fmaxf(m, lane_xor_low<2>(m));
    if (lpr > 4) m = fmaxf(m, lane_xor_low<4>(m));
    if (lpr > 8) m = fmaxf(m, lane_xor_low<8>(m));
    if (lpr > 16) { const float2 p2 = lane_pair<16>(m); m = fmaxf(p2.x, p2.y); }
    const float M = __shfl(m, lane - sl);  // the leader's max, to its group
    float l = 0.0f;
    if (act)
      for (int j = sl; j < nbv; j += lpr) l += rescaled(bst[j * a.R + row], M);
    l += lane_xor_low<1>(l);
    l += lane_xor_low<2>(l);
    if (lpr > 4) l += lane_xor_low<4>(l);
    if (lpr > 8) l += lane_xor_low<8>(l);
    if (lpr > 16) { const float2 p2 = lane_pair<16>(l); l = p2.x + p2.y; }
    if (act && sl == 0) publish_stat(row, M, l);
  }

  SDV_PHASE(3);
  // ------------------------------------------------------------------ 2. p.V
  const uint8_t* vlayer = a.v_pages + layer * a.v_ls;
  const float* slayer = a.v_scales + layer * a.s_ls;
  float* lparts = reinterpret_cast<float*>(smem + lay.parts);
  float2* lgs = reinterpret_cast<float2*>(smem + lay.gstats);  // per row: group (max, 1/sum)
  // the group's statistics: wavefront nt waits until all nvq items have published row tile nt, merges them
  // in a fixed order -- item slice j takes items j, j+nsl, ..., then a fixed tree -- and shares
  // (max, 1/sum) of each row through LDS, so every wavefront and workgroup of the group gets
  // identical values.  Every wavefront issues its first V loads before this wait (the
  // barrier at its end waits for them: the fence of __syncthreads covers global loads; an
  // LDS-only barrier there, letting them run under the probability pass, measured no faster,
  // as they have landed before the poll returns).  An
  // expired wait leaves (NaN, NaN): every probability, partial and output of the group is NaN.
  // A graph-recorded call reads the poison word with its first poll: on a poisoned workspace
  // (an earlier graph-recorded call expired, so statistics words carrying a recorded tag may be
  // left over) the call is refused the same way -- NaN statistics, NaN outputs, counted.
  auto group_stats = [&](float (&gm)[NT], float (&ginv)[NT]) {
    if (wave < NT) {  // wavefront nt polls and merges row tile nt (all tiles at once)
      // entries in flight per lane: a group has at most kFusedGroupItems = 32 items and a
      // slice at least a quarter of them
      constexpr int PB = 8;
      // lane = (item slice, row): 16 rows x 4 slices, or 8 x 8 when the rows fit in 8 and the
      // group has more than 8 items, so that more lanes share the merges (one layer at 8K, 64
      // items: 13.3 -> 12.8 us; with 4 or 5 items the extra tree level costs more than it saves)
      const bool narrow = NT == 1 && a.R <= 8 && nvq > 8;
      const int nsl = narrow ? 8 : 4;                      // item slices
      const int rl = narrow ? (lane & 7) : n, sl = narrow ? (lane >> 3) : g;
      const int ne = (nvq - sl + nsl - 1) / nsl;           // items of this slice (<= PB)
      {
        const int nt = wave;
        const int rr = nt * 16 + rl;
        const uint64_t* fp = fs + 2 * ((int64_t)item0 * 64 + (rr < a.R ? rr : 0));
        const uint64_t ready_word = (uint64_t)a.tag << 32;  // stands in for entries past the slice
        float mk[PB], lk[PB];
        const uint32_t poison =
            graph_call ? __hip_atomic_load(a.sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        bool expired = false;
        static_assert(kFusedGroupItems <= 4 * PB, "every slice's entries fit one poll round");
        {
          constexpr int k0 = 0;
          uint64_t em[PB], el[PB];
#pragma unroll
          for (int k = 0; k < PB; ++k) {
            const uint64_t* ep = fp + (int64_t)(sl + nsl * (k0 + k)) * 128;
            em[k] = k0 + k < ne ? load_dev_u64(ep) : ready_word;
            el[k] = k0 + k < ne ? load_dev_u64(ep + 1) : ready_word;
          }
          unsigned spins = 0;
          for (;;) {
            bool ready = true;
#pragma unroll
            for (int k = 0; k < PB; ++k) ready = ready && has_tag(em[k], a.tag) && has_tag(el[k], a.tag);
            if (__ballot(!ready) == 0 && a.spin_limit != 0) break;  // 0: give up at once (tests)
            if (++spins >= a.spin_limit) {
              expired = true;
              break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int k = 0; k < PB; ++k) {
              const uint64_t* ep = fp + (int64_t)(sl + nsl * (k0 + k)) * 128;
              if (!has_tag(em[k], a.tag)) em[k] = load_dev_u64(ep);
              if (!has_tag(el[k], a.tag)) el[k] = load_dev_u64(ep + 1);
            }
          }
#pragma unroll
          for (int k = 0; k < PB; ++k) {
            mk[k] = k0 + k < ne ? word_value(em[k]) : -INFINITY;
            lk[k] = k0 + k < ne ? word_value(el[k]) : 0.0f;
          }
        }
        // The row's max over all of the group's entries first (the lane tree of the sum below),
        // then each entry rescaled once against it and the rescaled sums added along the same
        // tree: one exp per entry and no branches, where a pairwise (max, sum) merge spends
        // two exps and a branch per merge level (one layer at 8K: 12.8 -> 12.4 us; one-layer
        // verify 16.3 -> 15.7 us)
        float m = mk[0];
#pragma unroll
        for (int k = 1; k < PB; ++k) m = fmaxf(m, mk[k]);
        if (narrow) m = fmaxf(m, lane_xor_low<8>(m));  // valid in the lanes with bit 3 clear
        float2 pm = lane_pair<16>(m);
        m = fmaxf(pm.x, pm.y);
        pm = lane_pair<32>(m);
        m = fmaxf(pm.x, pm.y);
        if (narrow)  // lanes with bit 3 set take the row's max from lane - 8
          m = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(m), __float_as_int(m), 0x118, 0xF, 0xF, false));
        float l = 0.0f;
#pragma unroll
        for (int k = 0; k < PB; ++k) l += mk[k] == -INFINITY ? 0.0f : lk[k] * fast_exp(mk[k] - m);
        if (narrow) l += lane_xor_low<8>(l);
        float2 pl = lane_pair<16>(l);
        l = pl.x + pl.y;
        pl = lane_pair<32>(l);
        l = pl.x + pl.y;
        if (expired || poison != 0) {  // wave-uniform (the poll loop exits on a ballot)
          m = l = __builtin_nanf("");
          if (lane == 0) s_fail = 1;
        }
        if (sl == 0 && rr < a.R) lgs[rr] = make_float2(m, 1.0f / l);
      }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int rr = nt * 16 + n;
      const float2 v = lgs[rr < a.R ? rr : 0];
      gm[nt] = v.x;
      ginv[nt] = v.y;
    }
  };

  // The probabilities, once per (row, token) for all wavefronts: the item's scores in LDS
  // become p = bf16(exp(s - M) / L) in place (with several row tiles a wavefront owns one
  // dimension tile of every block, so forming p inside the p.V loop would repeat every exp
  // once per tile).  Masked (-inf) scores give p = 0.  Needs the group statistics in LDS.
  auto prob_pass = [&]() {
    const int nvec = nbv * (kBlock / 8);  // 8-score vectors per row
    for (int e = tid; e < a.R * nvec; e += NTHR) {
      const int row = e / nvec, v = e - row * nvec;
      uint4* pp = reinterpret_cast<uint4*>(lsc + row * lrow + v * 8);
      const float2 st = lgs[row];
      const uint4 w4 = *pp;
      const uint32_t sw[4] = {w4.x, w4.y, w4.z, w4.w};
      float pr[8];
      // exp(s - M) as 2^(s log2 e - M log2 e), one FMA per score (28 layers at 8K, S=5: about
      // 0.5 us less VALU time than a subtract and a multiply)
      const float nml = -st.x * kLog2e;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float sc = (i & 1) ? bf16_hi(sw[i >> 1]) : bf16_lo(sw[i >> 1]);
        pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc, kLog2e, nml)) * st.y;  // -inf score -> 0
      }
      *pp = make_uint4(pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]), pack_bf16x2(pr[4], pr[5]),
                       pack_bf16x2(pr[6], pr[7]));
    }
  };

  float gm[NT], ginv[NT];
  if constexpr (kUnitPV) {
    // Units of (4 blocks, up to 4 dimension tiles); wavefront w takes units w, w + W, ...,
    // all of the same dimension tiles (W is a multiple of the units per stage), accumulates
    // them in registers and leaves its sum in its own LDS slot; the item's partial adds the
    // slots of each dimension tile in wavefront order.  The assignment is fixed, so the
    // partial is bitwise repeatable.
    constexpr int UT = DT < 4 ? DT : 4;  // 16-dimension tiles per unit
    constexpr int NH = DT / UT;          // units per stage of 4 blocks
    static_assert(W % NH == 0, "a wavefront's units cover the same dimension tiles");
    constexpr int UD = UT * 16;          // dimensions of a unit (an LDS slot row)
    const int nstage = (nbv + 3) >> 2;
    const int nunits = nstage * NH;
    struct Unit {
      uint4 code[UT];
      float scl;
      int nvalid;
    };
    auto load_u = [&](int u, Unit& x) {
      const int k = u / NH, hf = u - k * NH;
      const int jb = 4 * k + g;
      const int pb = (u < nunits && jb < nbv) ? lpb[jb] : -1;
      x.nvalid = pb >= 0 ? min(max(T - (tok0 + jb * kBlock), 0), kBlock) : 0;
      const int64_t page = (int64_t)(x.nvalid > 0 ? pb : 0) * a.KV + kvh;
      const uint8_t* vp = vlayer + (page * D + hf * UT * 16 + n) * kBlock;
#pragma unroll
      for (int t = 0; t < UT; ++t) x.code[t] = load_stream16(vp + t * 16 * kBlock);
      x.scl = __builtin_nontemporal_load(slayer + page * kBlock + n);
    };
    f32x4 accw[UT];  // this wavefront's dimension tiles, summed over its units
#pragma unroll
    for (int t = 0; t < UT; ++t) accw[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    auto compute_u = [&](int u, Unit& x) {
      const int k = u / NH;
      const int jb = 4 * k + g;
      if (__ballot(x.nvalid < kBlock) != 0) {  // wave-uniform: sanitize slots that are not tokens
        uint32_t bmask[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int kk2 = min(max(x.nvalid - 4 * w, 0), 4);
          bmask[w] = kk2 >= 4 ? 0xFFFFFFFFu : ((1u << (8 * kk2)) - 1u);
        }
#pragma unroll
        for (int t = 0; t < UT; ++t) {
          x.code[t].x &= bmask[0];
          x.code[t].y &= bmask[1];
          x.code[t].z &= bmask[2];
          x.code[t].w &= bmask[3];
        }
        x.scl = n < x.nvalid ? x.scl : 0.0f;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // the probabilities of the block (formed once in LDS); rows past R and lane groups
        // past the item take p = 0 (never inf * 0)
        uint4 w4 = make_uint4(0u, 0u, 0u, 0u);
        if (jb < nbv && n < a.R) w4 = *reinterpret_cast<const uint4*>(lsc + n * lrow + jb * kBlock + 8 * h);
        const bf16x8 pop = __builtin_bit_cast(bf16x8, w4);
        float sv[8];
        if (h == 0) {
          sv[0] = row_bcast<0>(x.scl); sv[1] = row_bcast<1>(x.scl); sv[2] = row_bcast<2>(x.scl);
          sv[3] = row_bcast<3>(x.scl); sv[4] = row_bcast<4>(x.scl); sv[5] = row_bcast<5>(x.scl);
          sv[6] = row_bcast<6>(x.scl); sv[7] = row_bcast<7>(x.scl);
        } else {
          sv[0] = row_bcast<8>(x.scl); sv[1] = row_bcast<9>(x.scl); sv[2] = row_bcast<10>(x.scl);
          sv[3] = row_bcast<11>(x.scl); sv[4] = row_bcast<12>(x.scl); sv[5] = row_bcast<13>(x.scl);
          sv[6] = row_bcast<14>(x.scl); sv[7] = row_bcast<15>(x.scl);
        }
#pragma unroll
        for (int t = 0; t < UT; ++t) {
          const uint32_t lo = h ? x.code[t].z : x.code[t].x;
          const uint32_t hi = h ? x.code[t].w : x.code[t].y;
          const f32x2 f01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
          const f32x2 f23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
          const f32x2 f45 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
          const f32x2 f67 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
          const bf16x8 vop = __builtin_bit_cast(
              bf16x8, make_uint4(pack_bf16x2(f01.x * sv[0], f01.y * sv[1]), pack_bf16x2(f23.x * sv[2], f23.y * sv[3]),
                                 pack_bf16x2(f45.x * sv[4], f45.y * sv[5]), pack_bf16x2(f67.x * sv[6], f67.y * sv[7])));
          accw[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop, accw[t], 0, 0, 0);
        }
      }
    };
    // two units in flight per wavefront, the last ones peeled (as in q.k^T); the first unit
    // is loaded before the group statistics wait, except by the polling wavefront of items of
    // kPollAfterMinBlocks blocks or more: its poll would return only after that load, which
    // queues behind the other workgroups' K streams (24-layer draft at 8K, 103-block items:
    // 21.4 -> 21.0 us; 28 layers equal; one-layer calls with 16-block items 0.15 us slower)
    constexpr int kPollAfterMinBlocks = 64;
    const bool poller_late = wave < NT && a.f_maxblk >= kPollAfterMinBlocks;  // wave-uniform
    Unit ua, ub;
    const int nsu = wave < nunits ? (nunits - 1 - wave) / W + 1 : 0;  // units wave, wave + W, ...
    if (nsu > 0 && !poller_late) load_u(wave, ua);
    group_stats(gm, ginv);
    if (nsu > 0 && poller_late) load_u(wave, ua);
    SDV_PHASE(4);
    // p formed once per (row, token) before the loop: a unit covers half the dimensions of
    // its blocks, so forming p per unit would repeat every exp (28 layers at 8K: 39.2 ->
    // 37.2 us together with the single-exit loops)
    prob_pass();
    __syncthreads();
    if (nsu > 0) {
      int s = 0;
      while (s + 2 < nsu) {
        load_u(wave + (s + 1) * W, ub);
        compute_u(wave + s * W, ua);
        load_u(wave + (s + 2) * W, ua);
        compute_u(wave + (s + 1) * W, ub);
        s += 2;
      }
      if (s + 1 < nsu) {
        load_u(wave + (s + 1) * W, ub);
        compute_u(wave + s * W, ua);
        compute_u(wave + (s + 1) * W, ub);
      } else {
        compute_u(wave + s * W, ua);
      }
    }
    // lane (g, n) holds row n, dims (wave % NH)*UD + t*16 + 4g .. +3; wavefronts w < nunits
    // have units
    if (nsu > 0 && n < a.R) {
#pragma unroll
      for (int t = 0; t < UT; ++t) *reinterpret_cast<f32x4*>(lparts + ((wave * a.R + n) * UD + t * 16 + 4 * g)) = accw[t];
    }
    __syncthreads();
    SDV_PHASE(5);
    // the item's partial: the slots of each dimension tile's wavefronts summed in wavefront order
    const int wu = min(W, nunits);  // wavefronts with units
    for (int o4 = tid; o4 * 4 < a.R * D; o4 += NTHR) {
      const int row = (4 * o4) / D, d = 4 * o4 - row * D, hf = d / UD, dl = d - hf * UD;
      f32x4 v = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
      for (int w = hf; w < wu; w += NH) v += *reinterpret_cast<const f32x4*>(lparts + ((w * a.R + row) * UD + dl));
      __builtin_amdgcn_raw_buffer_store_b128(part_enc(v), prs, (int)((item * pstride + 4 * o4) * 4), 0, 16);
    }
  } else {
    // wavefront (tile group tg, part pt): dims [tg*DTW*16, +DTW*16), blocks [pbeg, pend)
    const int tg = wave % NTG, pt = wave / NTG;
    const int pbeg = (nbv * pt) / TP, pend = (nbv * (pt + 1)) / TP;
    const int nstage = (pend - pbeg + 3) >> 2;  // 4 blocks per stage (lane group g: block 4*st + g)
    struct Stage {
      uint4 code[DTW];
      float scl;
      int nvalid;
    };
    auto load_v = [&](int st, Stage& s) {
      const int jb = pbeg + 4 * st + g;
      const int pb = jb < pend ? lpb[min(jb, nbv - 1)] : -1;
      s.nvalid = pb >= 0 ? min(max(T - (tok0 + jb * kBlock), 0), kBlock) : 0;
      const int64_t page = (int64_t)(s.nvalid > 0 ? pb : 0) * a.KV + kvh;
      const uint8_t* vp = vlayer + (page * D + tg * DTW * 16 + n) * kBlock;
  #pragma unroll
      for (int dtw = 0; dtw < DTW; ++dtw) s.code[dtw] = load_stream16(vp + dtw * 16 * kBlock);
      s.scl = __builtin_nontemporal_load(slayer + page * kBlock + n);
    };
    // kVStages stages of V in flight per wavefront (3 with wider tiles): a stage is only 1 KiB
    // of codes per 16-dim tile, so a deep ring keeps enough bytes moving
    constexpr int SD = DTW >= 2 ? 3 : kVStages;
    Stage ring[SD];
    // With items of kPollFirstMinBlocks blocks or more the polling wavefronts load their
    // ring only after the group statistics: a poll load queued behind the ring returns once
    // the ring has (first poll check 3.2 us after the publish against 1.6 us for decode; 28
    // layers at 8K: 48.8-49.5 -> 47.7-47.8 us).  Small items lose by it (one layer: +0.9
    // us): their wait is short and their ring is most of their p.V.
    constexpr int kPollFirstMinBlocks = 32;
    const bool poll_first = a.f_maxblk >= kPollFirstMinBlocks;  // workgroup-uniform
    if (!poll_first || wave >= NT) {  // wave-uniform
  #pragma unroll
      for (int i = 0; i < SD; ++i)
        if (i < nstage) load_v(i, ring[i]);
    }
    group_stats(gm, ginv);
    SDV_PHASE(4);
    if (poll_first && wave < NT) {
  #pragma unroll
      for (int i = 0; i < SD; ++i)
        if (i < nstage) load_v(i, ring[i]);
    }
    prob_pass();
    __syncthreads();
    f32x4 acc[DTW][NT];
  #pragma unroll
    for (int dtw = 0; dtw < DTW; ++dtw)
  #pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[dtw][nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    auto compute_v = [&](int st, Stage& s) {
      const int jb = pbeg + 4 * st + g;
      const bool in_part = jb < pend;
      if (__ballot(s.nvalid < kBlock) != 0) {  // wave-uniform: sanitize slots that are not tokens
        uint32_t bmask[4];
  #pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int k = min(max(s.nvalid - 4 * w, 0), 4);
          bmask[w] = k >= 4 ? 0xFFFFFFFFu : ((1u << (8 * k)) - 1u);
        }
  #pragma unroll
        for (int dtw = 0; dtw < DTW; ++dtw) {
          s.code[dtw].x &= bmask[0];
          s.code[dtw].y &= bmask[1];
          s.code[dtw].z &= bmask[2];
          s.code[dtw].w &= bmask[3];
        }
        s.scl = n < s.nvalid ? s.scl : 0.0f;
      }
  #pragma unroll
      for (int h = 0; h < 2; ++h) {
        bf16x8 pop[NT];
  #pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          // rows past R and lane groups past the part take p = 0 (never inf * 0)
          const int row = nt * 16 + n;
          uint4 w4 = make_uint4(0u, 0u, 0u, 0u);
          if (in_part && row < a.R) w4 = *reinterpret_cast<const uint4*>(lsc + row * lrow + jb * kBlock + 8 * h);
          pop[nt] = __builtin_bit_cast(bf16x8, w4);
        }
        float sv[8];
        if (h == 0) {
          sv[0] = row_bcast<0>(s.scl); sv[1] = row_bcast<1>(s.scl); sv[2] = row_bcast<2>(s.scl);
          sv[3] = row_bcast<3>(s.scl); sv[4] = row_bcast<4>(s.scl); sv[5] = row_bcast<5>(s.scl);
          sv[6] = row_bcast<6>(s.scl); sv[7] = row_bcast<7>(s.scl);
        } else {
          sv[0] = row_bcast<8>(s.scl); sv[1] = row_bcast<9>(s.scl); sv[2] = row_bcast<10>(s.scl);
          sv[3] = row_bcast<11>(s.scl); sv[4] = row_bcast<12>(s.scl); sv[5] = row_bcast<13>(s.scl);
          sv[6] = row_bcast<14>(s.scl); sv[7] = row_bcast<15>(s.scl);
        }
  #pragma unroll
        for (int dtw = 0; dtw < DTW; ++dtw) {
          const uint32_t lo = h ? s.code[dtw].z : s.code[dtw].x;
          const uint32_t hi = h ? s.code[dtw].w : s.code[dtw].y;
          const f32x2 f01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
          const f32x2 f23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
          const f32x2 f45 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
          const f32x2 f67 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
          const bf16x8 vop = __builtin_bit_cast(
              bf16x8, make_uint4(pack_bf16x2(f01.x * sv[0], f01.y * sv[1]), pack_bf16x2(f23.x * sv[2], f23.y * sv[3]),
                                 pack_bf16x2(f45.x * sv[4], f45.y * sv[5]), pack_bf16x2(f67.x * sv[6], f67.y * sv[7])));
  #pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[dtw][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[nt], acc[dtw][nt], 0, 0, 0);
        }
      }
    };
    // Full rounds (every reload a stage of the part) in a loop with one exit, at the head:
    // every path into the head has the ring's loads pending in ring order, so stage i waits
    // only for its own loads (a break after stage i would reorder the pending loads of the
    // merged paths and make the compiler wait for nearly the whole ring).  The last (up to
    // 2 * SD - 1) stages follow the loop with no loads past the part, which the barrier after
    // p.V would otherwise wait for (one-layer verify at 8K: 16.7 -> 16.3 us).
    int st0 = 0;
    for (; st0 + 2 * SD <= nstage; st0 += SD) {  // every reload is a stage of the part
  #pragma unroll
      for (int i = 0; i < SD; ++i) {
        compute_v(st0 + i, ring[i]);
        load_v(st0 + i + SD, ring[i]);
      }
    }
  #pragma unroll
    for (int i = 0; i < SD; ++i) {
      if (st0 + i < nstage) {  // wave-uniform
        compute_v(st0 + i, ring[i]);
        if (st0 + i + SD < nstage) load_v(st0 + i + SD, ring[i]);
      }
    }
  #pragma unroll
    for (int i = 0; i < SD; ++i)
      if (st0 + SD + i < nstage) compute_v(st0 + SD + i, ring[i]);

    // lane (g, n) holds rows nt*16+n, dims tg*DTW*16 + dtw*16 + 4g .. +3; with several block
    // parts every part goes to its LDS slot and all threads add the slots in part order (the
    // two part-0 wavefronts adding the others alone took 0.95 us after p.V on 28-layer verify)
    if (TP > 1) {
      __syncthreads();  // the parts overwrite the probabilities the other wavefronts read
  #pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int row = nt * 16 + n;
        if (row < a.R) {
  #pragma unroll
          for (int dtw = 0; dtw < DTW; ++dtw)
            *reinterpret_cast<f32x4*>(lparts + ((pt * a.R + row) * D + tg * DTW * 16 + dtw * 16 + 4 * g)) = acc[dtw][nt];
        }
      }
    }
    // every wavefront is past its statistics before any partial is published (an owner that
    // has seen all partials clears the statistics)
    __syncthreads();
    SDV_PHASE(5);
    if (TP > 1) {
      for (int o4 = tid; o4 * 4 < a.R * D; o4 += NTHR) {
        f32x4 v = *reinterpret_cast<const f32x4*>(lparts + 4 * o4);
  #pragma unroll
        for (int p2 = 1; p2 < TP; ++p2) v += *reinterpret_cast<const f32x4*>(lparts + p2 * a.R * D + 4 * o4);
        __builtin_amdgcn_raw_buffer_store_b128(part_enc(v), prs, (int)((item * pstride + 4 * o4) * 4), 0, 16);
      }
    } else {
  #pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int row = nt * 16 + n;
        if (row < a.R) {
  #pragma unroll
          for (int dtw = 0; dtw < DTW; ++dtw) {
            const int d0 = tg * DTW * 16 + dtw * 16 + 4 * g;
            __builtin_amdgcn_raw_buffer_store_b128(part_enc(acc[dtw][nt]), prs,
                                                   (int)((item * pstride + (int64_t)row * D + d0) * 4), 0, 16);
          }
        }
      }
    }
  }

  SDV_PHASE(6);
  // ------------------------------------------------------------------ 3. output
  // Workgroup c < nvq of the group owns output chunks [lo, lo + w) (16 bytes each) and sums
  // them over the group's items.  Partial words are never 0 once written, and every item's
  // slot was zeroed before that item published the statistics this workgroup took, so the
  // owner polls the data itself.  Each chunk gets a group of P2 lanes (P2 = nvq rounded up to a
  // power of two): lane i of the group loads item i's chunk, and a fixed butterfly over the
  // group (quad permutes, row shifts, row and half-wave pairs) leaves the sum in its first
  // lane, which writes the BF16 output -- no LDS round trips and no barrier between polling
  // and the output (against a two-level sum through LDS: one layer at 8K 12.3 -> 11.75 us, at
  // 2K 10.5 -> 9.8 us).
  // Having seen every item's chunks the owner knows that every workgroup of the group is past
  // its statistics: it clears its share of them, leaving the statistics area zero for the
  // next call (the replays of a graph reuse their tag).
  static_assert(kFusedGroupItems <= 32, "a chunk's items fit half a wavefront");
  const int P2 = nvq <= 1 ? 1 : nvq <= 2 ? 2 : nvq <= 4 ? 4 : nvq <= 8 ? 8 : nvq <= 16 ? 16 : 32;
  const int nsl_out = w * P2;  // lane slots: chunk o = slot / P2, item slot % P2
  __syncthreads();  // the item's own partial stores have completed
  // Up to kOutLoads slots per thread are loaded before any is polled (verify: 960 chunks per
  // owner), so the rounds do not wait for each other.
  constexpr int kOutLoads = 4;
  for (int e0 = 0; e0 < nsl_out; e0 += NTHR * kOutLoads) {  // workgroup-uniform
    u32x4_t v[kOutLoads];
    int off[kOutLoads];
#pragma unroll
    for (int r = 0; r < kOutLoads; ++r) {
      const int e = e0 + r * NTHR + tid;
      const int o = e / P2, cc = e - o * P2;
      const bool act = e < nsl_out && cc < nvq;
      off[r] = act ? (int)(((int64_t)(item0 + cc) * pstride + 4 * (lo + o)) * 4) : 0;
      v[r] = (u32x4_t){1u, 1u, 1u, 1u};  // decodes to 0
      if (act) v[r] = __builtin_amdgcn_raw_buffer_load_b128(prs, off[r], 0, 16);
    }
    unsigned spins = 0;
    for (;;) {
      bool ready = true;
#pragma unroll
      for (int r = 0; r < kOutLoads; ++r) ready = ready && v[r][0] != 0u && v[r][1] != 0u && v[r][2] != 0u && v[r][3] != 0u;
      if (__ballot(!ready) == 0 && a.spin_limit != 0) break;  // 0: give up at once (tests)
      if (++spins >= a.spin_limit) {
        if (lane == 0) s_fail = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int r = 0; r < kOutLoads; ++r)
        if (!(v[r][0] != 0u && v[r][1] != 0u && v[r][2] != 0u && v[r][3] != 0u))
          v[r] = __builtin_amdgcn_raw_buffer_load_b128(prs, off[r], 0, 16);
    }
#pragma unroll
    for (int r = 0; r < kOutLoads; ++r) {
      if (e0 + r * NTHR >= nsl_out) break;  // workgroup-uniform
      float4 f = part_dec(v[r]);
      // the sum lands in the group's first lane (the row shifts serve the lanes whose bit is
      // clear, the first lane among them)
      auto level = [&](auto xfer) { f.x += xfer(f.x); f.y += xfer(f.y); f.z += xfer(f.z); f.w += xfer(f.w); };
      if (P2 > 1) level([](float x) { return lane_xor_low<1>(x); });
      if (P2 > 2) level([](float x) { return lane_xor_low<2>(x); });
      if (P2 > 4) level([](float x) { return lane_xor_low<4>(x); });
      if (P2 > 8) level([](float x) { return lane_xor_low<8>(x); });
      if (P2 > 16) {
        const float2 px = lane_pair<16>(f.x), py = lane_pair<16>(f.y), pz = lane_pair<16>(f.z), pw = lane_pair<16>(f.w);
        f = make_float4(px.x + px.y, py.x + py.y, pz.x + pz.y, pw.x + pw.y);
      }
      const int e = e0 + r * NTHR + tid;
      const int o = e / P2;
      if (e - o * P2 == 0 && e < nsl_out) {
        const int o4 = lo + o;
        const int row = (4 * o4) / D, d = 4 * o4 - row * D, hl = row / a.S, si = row % a.S;
        uint16_t* dst = a.out + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + d;
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(f.x, f.y), pack_bf16x2(f.z, f.w));
      }
    }
  }
  __syncthreads();
  SDV_PHASE(7);
  // a wait of this workgroup expired: its outputs become NaN, the error is counted (and a
  // graph-recorded call poisons the workspace), and nothing is cleared
  if (s_fail) {
    nan_slice();
    if (tid == 0) {
      count_sync_error(a);
      if (graph_call) __hip_atomic_store(a.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  SDV_PHASE(8);
  if (c < nown) {
    for (int e = c + tid * nown; e < nvq * a.R; e += NTHR * nown) {
      uint64_t* p = fs + 2 * ((int64_t)(item0 + e / a.R) * 64 + e % a.R);
      store_dev_u64(p, 0);
      store_dev_u64(p + 1, 0);
    }
  }
  SDV_PHASE(9);
  SDV_PHASE_FLUSH();
}


__global__ void zero_kernel(uint32_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

// ---------------------------------------------------------------------------- prefill
// Shapes with more query rows than one row-tile group holds (R = G*S > 64: prefill and
// chunked-prefill blocks, model_self.py:471-504, 637-648) in two launches whose workspace holds
// the per-row (max, sum) of each key part -- 8 bytes per row and part -- and V dequantized once
// (2 bytes per key and dimension of each KV head) instead of the O(S*T) scores:
//   pass 1  each wavefront takes 32 rows (two MFMA row tiles) and streams one part of the page
//           blocks its rows can see (one workgroup per part): S^T = K Q^T on MFMA (the K page is
//           the A operand, the rows the B operand; one K operand serves both tiles), scores
//           rounded to BF16 twice, offset-causal mask, online (max, sum) per lane, merged over
//           the lane groups into the part's (max, sum) per row.  The launch also dequantizes
//           V, each stage of two blocks once, as bf16(fp32(code) * scale) in the lane order of
//           pass 2's MFMA operand.
//   pass 2  merges the parts in part order into (M, L); each wavefront (32 rows) streams its
//           part of the blocks again, recomputes its rows' BF16 scores and forms
//           p = bf16(exp(s - M) / L) in registers.  A lane's S^T fragment (row n, tokens
//           4g..4g+3 of each of two blocks) is exactly the B operand of O^T = V_hat^T P^T with
//           those 8 tokens as its k-slots; the A operand is the dequantized V of the two
//           blocks, 16 bytes per lane and dimension tile.  O^T accumulates in fp32; the parts'
//           partials are summed in part order by the last part to finish, and leave as BF16,
//           four dimensions of one row per lane.
// Both passes stream stages of four blocks whose K (and dequantized V) the workgroup's four
// wavefronts load once and share through LDS, one barrier per stage.
// Rows are head-major (row r: head r / S, token r % S) as in the other kernels.  Row r sees
// keys j <= T - S + r % S (the eager mask); T >= S is the caller's contract (the S new tokens
// are part of the context), and a row that sees no key outputs 0.  The page ids of the
// workgroup's blocks are staged in LDS, kPrefillWindow at a time.  Measured steps (2048 x 8192,
// 12/2/128 and 14/2/64, both passes): 451 / 324 us with 16 rows per wavefront and V dequantized
// per stage into LDS by the workgroup; scalar branches for the unmasked stages 442 / 281;
// two row tiles in pass 1 382 / 263; two in pass 2 350 / 235; V dequantized by pass 1 and
// MFMA results in VGPRs 332 / 218; 16-byte part slots and key parts per launch size 303 / 196;
// each stage's K and V loaded once per workgroup and shared through LDS 284 / 182; stages of
// four blocks, products issued by phase 271 / 173; v_max3 for the stage max and register
// budgets held per pass 265 / 171; constant block indices in the loads and 1/L folded into
// the exponent 258 / 167 (worst rel-L2 per 64-row block against eager 1.8e-4 -> 2.3e-4); pass
// 2's statistics loads eight parts at a time 253 / 160.
constexpr int kPrefillRows = 16;   // query rows per MFMA row tile
constexpr int kPass1Waves = 4;     // wavefronts per workgroup, pass 1
constexpr int kPass2Waves = 4;     // and pass 2
constexpr int prefill_waves(bool OUT) { return OUT ? kPass2Waves : kPass1Waves; }
constexpr int kPrefillWindow = 256;   // page ids staged in LDS per round
constexpr int kStageBlocks = 4;      // page blocks per stage (a multiple of 2 dividing the window)
// Pass 1: row tiles per wavefront (each K operand it loads serves this many tiles; 2048 x 8192,
// pass 1 with one tile 158 / 93 us (12/2/128 / 14/2/64), with two 101 / 77 us)
constexpr int kPass1Tiles = 2;
// Pass 2: row tiles per wavefront, and the rows of a workgroup (a row group: its part slots,
// its counter)
constexpr int kPass2Tiles = 2;
constexpr int kPass2Rows = kPass2Tiles * kPrefillRows * kPass2Waves;
// Both passes split each row group's keys in parts, one workgroup each (pass 2 merges pass 1's
// (max, sum) in part order; the last pass-2 part to finish sums the parts' outputs), as many
// as bring the launch to about this many workgroups, at most kPrefillMaxParts and none under
// 8 blocks.  Pass 1: 2048 x 8192 in 8 parts (12/2/128: 101 us, 16 parts 108 us; 14/2/64: 74 us,
// 11 parts 83 us, 6 parts 80 us);
// pass 2: one round, two wavefronts per SIMD for head_dim 128 and three for 64 (2048 x 8192: 2
// parts 12/2/128, 3 parts 14/2/64).
constexpr int pass1_workgroups(int D) { return D == 128 ? 1536 : 1792; }
constexpr int pass2_workgroups(int D) { return D == 128 ? 512 : 768; }
constexpr int kPrefillMaxParts = 64;
// pass 2: the last part to finish adds every part's slot of its row group
constexpr int kPrefillMaxParts2 = 8;

// Resident wavefronts per SIMD the register budget is held to: pass 1 four (at most 128
// VGPRs), pass 2 three for head_dim 64 (168) and two for 128 (its 64 fp32 accumulators per lane).
constexpr int prefill_waves_per_simd(int D, bool OUT) { return !OUT ? 4 : D == 64 ? 3 : 2; }

// Pass 2's parts of row group k (0-based within its head) when they follow its key count:
// the group's last row sees keys up to T - S + min(S, rows * (k + 1)) - 1, in blocks of 16, cut
// into parts of at most kstar blocks.  The host plans with T = max_seq_len; the kernel maps
// its workgroups with the same arguments, so both agree on the grid.
__host__ __device__ inline int pass2_group_parts(int k, int S, int T, int rows, int kstar) {
  const int keys = T - S + min(S, rows * (k + 1));
  const int blocks = keys > 0 ? (keys + kBlock - 1) / kBlock : 0;
  return max(1, (blocks + kstar - 1) / kstar);
}

template <int D, bool OUT>
__global__ __launch_bounds__(64 * prefill_waves(OUT)) __attribute__((amdgpu_waves_per_eu(prefill_waves_per_simd(D, OUT))))
void prefill_kernel(AttnArgs a) {
  // row tiles of 16 rows per wavefront (two in both passes: each K operand a wavefront reads
  // serves 32 rows)
  constexpr int KK = D / 32, DT = D / 16, NT = OUT ? kPass2Tiles : kPass1Tiles, ROWS = NT * 16;
  constexpr int W = prefill_waves(OUT);
  constexpr int DTW = DT / W;  // pass 1: dimension tiles of V each wavefront dequantizes
  static_assert(OUT || DTW * W == DT, "the wavefronts share the dimension tiles evenly");
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  __shared__ int lpb[kPrefillWindow];
  __shared__ int s_kend;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int kvh = blockIdx.y, zb = blockIdx.z, b = zb % a.B, layer = zb / a.B;
  const int T = seq_len_of(a, b);
  const int grp = zb * a.KV + kvh;
  // the keys of a row group are split in parts, one workgroup each: a.pf_split in pass 1,
  // a.pf_parts in pass 2
  int nparts = OUT ? a.pf_parts : a.pf_split;
  int split = (int)(blockIdx.x % nparts);
  int rgi = (int)(blockIdx.x / nparts);
  if (OUT && a.pf_kstar > 0) {  // parts per row group by its key count: head h, then group k
    const int rgph = a.S / kPass2Rows;
    const int h = (int)blockIdx.x / a.pf_wh;
    int off = (int)blockIdx.x - h * a.pf_wh, k = 0;
    for (; k < rgph - 1; ++k) {
      const int pk = pass2_group_parts(k, a.S, a.max_seq_len, kPass2Rows, a.pf_kstar);
      if (off < pk) break;
      off -= pk;
    }
    nparts = pass2_group_parts(k, a.S, a.max_seq_len, kPass2Rows, a.pf_kstar);
    split = off;
    rgi = h * rgph + k;
  }
  const int row0 = (rgi * W + wave) * ROWS;

  // this lane's rows (row tile nt: row row0 + nt*16 + n): q operand and last visible key
  bf16x8 qop[NT][KK];
  int lim[NT];
  bool rv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = row0 + nt * 16 + n;
    rv[nt] = r < a.R;
    const int hl = rv[nt] ? r / a.S : 0, si = rv[nt] ? r % a.S : 0;
    const uint16_t* qp = a.q + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + g * 8;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qop[nt][kk] = rv[nt] ? load_bf16x8(qp + kk * 32) : zero_bf16x8();
    lim[nt] = rv[nt] ? min(T - 1, T - a.S + si) : -1;
  }
  // blocks this wavefront streams (keys 0 .. max lim) and the smallest lim of its rows (every
  // key up to it is seen by every row: the blocks below nfull need no mask).  Both are
  // wave-uniform and kept in scalar registers, so that every branch on them below is a
  // scalar branch rather than a change of the execution mask.
  int kend = 0, kmin = INT_MAX;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    kend = max(kend, lim[nt] + 1);
    kmin = min(kmin, rv[nt] ? lim[nt] : INT_MAX);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    kend = max(kend, __shfl_xor(kend, off));
    kmin = min(kmin, __shfl_xor(kmin, off));
  }
  const int nblk = __builtin_amdgcn_readfirstlane((kend + kBlock - 1) >> 4);
  const int nfull = __builtin_amdgcn_readfirstlane(kmin == INT_MAX ? 0 : max(0, (kmin + 1) >> 4));
  if (tid == 0) s_kend = 0;
  __syncthreads();
  if (lane == 0) atomicMax(&s_kend, nblk);
  __syncthreads();
  const int nblk_wg = __builtin_amdgcn_readfirstlane(s_kend);

  // page addressing: a page id's base is scalar (this layer and KV head), the lane's offset a
  // 32-bit vector offset
  const uint16_t* klayer = a.k_pages + layer * a.k_ls + (int64_t)kvh * (kBlock * D);
  const uint8_t* vlayer = a.v_pages + layer * a.v_ls + (int64_t)kvh * (D * kBlock);
  const float* slayer = a.v_scales + layer * a.s_ls + (int64_t)kvh * kBlock;
  const int64_t kpage = (int64_t)a.KV * (kBlock * D);  // K elements, V bytes per page id
  const int64_t spage = (int64_t)a.KV * kBlock;        // scales per page id
  const unsigned koff = (unsigned)lane * 8u;
  const unsigned voff = (unsigned)((wave * DTW * 16 + n) * kBlock + 4 * g);
  const int* btrow = a.block_table + (int64_t)b * a.max_blocks;
  float2* st = a.stats + (int64_t)grp * a.R * a.pf_split;  // row r, pass-1 part k: st[r * a.pf_split + k]
  // this workgroup's key blocks: part `split` of [0, nblk_wg)
  const int part = (((nblk_wg + nparts - 1) / nparts) + kStageBlocks - 1) & ~(kStageBlocks - 1);  // whole stages
  const int blo = min(nblk_wg, split * part);
  const int bhi = min(nblk_wg, blo + part);

  // Scores in the eager units: bf16(bf16(x) / sqrt(D)).  For head_dim 64 the divisor is 8 and
  // bf16(x) * 0.125 is exact, so the scores are kept as bf16(x) -- one rounding -- and the
  // factor 0.125 goes into the row max (exact) and into the exponent's coefficient
  // (kLog2e * 0.125 is exact, so fma(bf16(x), kLog2e * 0.125, c) is bit for bit
  // fma(bf16(x) * 0.125, kLog2e, c)).
  constexpr float kUnit = D == 64 ? 0.125f : 1.0f;
  constexpr float kExpCoef = kLog2e * kUnit;
  const float csc = a.inv_sqrt_d;
  auto eager4 = [&](const f32x4& s, float* y) {
    if constexpr (D == 64) {
      const uint32_t r01 = pack_bf16x2(s[0], s[1]), r23 = pack_bf16x2(s[2], s[3]);
      y[0] = bf16_lo(r01);
      y[1] = bf16_hi(r01);
      y[2] = bf16_lo(r23);
      y[3] = bf16_hi(r23);
    } else {
      float t[4];
      round_scaled4(s[0], s[1], s[2], s[3], csc, t);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = t[i];
    }
  };

  float m_run[NT], l_run[NT];   // pass 1: running max and sum
  float nml[NT];                // pass 2: -M log2 e - log2 L per row
  f32x4 acc[DT][NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.0f;
    nml[nt] = 0.0f;
    if (OUT && rv[nt]) {
      // (M, L) of the row: its parts merged in part order
      const float2* sr = st + (int64_t)(row0 + nt * 16 + n) * a.pf_split;
      // eight parts' loads in flight at a time, merged in part order
      float m = -INFINITY, l = 0.0f;
      for (int k0 = 0; k0 < a.pf_split; k0 += 8) {
        float2 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = k0 + i < a.pf_split ? sr[k0 + i] : make_float2(-INFINITY, 0.0f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (k0 + i == 0) {
            m = v[0].x;
            l = v[0].y;
          } else {
            merge_fast(m, l, v[i].x, v[i].y);
          }
        }
      }
      if (l > 0.0f) {
        // p = exp(s - M) / L as one exp2: 2^(s log2 e - M log2 e - log2 L) (v_log_f32 is within
        // 1 ulp; |log2 L| <= log2 T, so p moves by ~1e-6 relative, far below its BF16 step)
        nml[nt] = -m * kLog2e - __builtin_amdgcn_logf(l);
      }
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt][nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  }

  // A stage is kStageBlocks = 4 consecutive blocks u = 0..3.  Its K operands (4 x KK chunks of
  // 1 KiB: block u, 32-dimension slice kk, in the lane order of the MFMA's A operand) and, for
  // pass 2, its dequantized V operand (2 x DT chunks of 1 KiB: pair h of blocks, dimension tile
  // dt, written by pass 1) are the same for every row, so the workgroup loads each chunk once
  // and shares it through LDS: wavefront w loads chunks w, w + W, ... of stage s + 2 into
  // registers while the workgroup computes stage s, and writes them to the LDS buffer of stage
  // s right after the barrier of stage s + 1.  One barrier per stage publishes the stage and
  // frees the other buffer.  Within a stage the q.k^T products of all four blocks go out
  // first, then the scores, then the p.V products: the MFMA unit has independent work while
  // the VALU rounds.
  constexpr int SB = kStageBlocks;
  constexpr int NKC = SB * KK, NC = NKC + (OUT ? (SB / 2) * DT : 0), CPW = NC / W;
  static_assert(CPW * W == NC && NKC % W == 0, "the wavefronts share the chunks evenly");
  __shared__ uint4 ring[2][NC * 64];
  const uint4* vh_grp = a.vhat + (int64_t)grp * a.vh_stages * (DT * 64) + lane;
  for (int w0 = blo; w0 < bhi; w0 += kPrefillWindow) {  // workgroup-uniform
    const int wn = min(kPrefillWindow, bhi - w0);
    __syncthreads();  // the previous window's page ids are no longer read
    for (int j = tid; j < wn; j += 64 * W) {
      const int pb = btrow[w0 + j];
      lpb[j] = (pb >= 0 && pb < a.num_blocks) ? pb : -1;
    }
    __syncthreads();
    const int jn = max(0, min(nblk - w0, wn));  // this wavefront's blocks in the window
    const int nst = (wn + SB - 1) / SB;         // the workgroup's stages in the window
    // page id of block jb of the window (jb < wn; the same word in every lane)
    auto page = [&](int jb) { return __builtin_amdgcn_readfirstlane(lpb[jb]); };
    uint4 stg[CPW];  // this wavefront's chunks of the next stage
    auto fetch = [&](int s4) {
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const int c = j * W + wave;
        if (j < NKC / W) {  // a K chunk: block u, slice kk; past the window, page 0 (never used)
          // u is a constant when every wavefront's chunk j falls in the same block
          const int u = KK % W == 0 ? (j * W) / KK : c / KK, kk = c - u * KK;
          const int jb = SB * s4 + u;
          const int pb = __builtin_amdgcn_readfirstlane(lpb[min(jb, kPrefillWindow - 1)]);
          const int64_t pg = jb < wn ? max(pb, 0) : 0;
          stg[j] = load_stream16(klayer + pg * kpage + (koff + kk * 512u));
        } else {            // a dequantized V chunk: pair h, dimension tile dt
          const int h = DT % W == 0 ? (j * W - NKC) / DT : (c - NKC) / DT, dt = (c - NKC) - h * DT;
          const int sg = min((w0 >> 1) + (SB / 2) * s4 + h, a.vh_stages - 1);
          stg[j] = vh_grp[(int64_t)sg * (DT * 64) + dt * 64];
        }
      }
    };
    auto stash = [&](int s4) {
#pragma unroll
      for (int j = 0; j < CPW; ++j) ring[s4 & 1][(j * W + wave) * 64 + lane] = stg[j];
    };
    auto compute_stage = [&](int s4, const uint4* sb) {
      const int jb0 = SB * s4, jg0 = w0 + jb0;  // window and global block of u = 0
      int pb[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) pb[u] = jb0 + u < jn ? page(jb0 + u) : -1;
      // scalar: every key of the stage exists, is valid and is seen by every row
      bool full = jg0 + SB <= nfull && jb0 + SB <= jn;
#pragma unroll
      for (int u = 0; u < SB; ++u) full = full && pb[u] >= 0;
      // q.k^T of the stage's blocks, all issued before any score is rounded
      f32x4 sacc[SB][NT];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const bf16x8 kop = __builtin_bit_cast(bf16x8, sb[(u * KK + kk) * 64 + lane]);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            sacc[u][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[nt][kk], kk == 0 ? (f32x4){0.0f, 0.0f, 0.0f, 0.0f} : sacc[u][nt], 0, 0, 0);
        }
      float y[NT][4 * SB];  // the stage's scores (in units of kUnit): block u in 4u .. 4u+3
#pragma unroll
      for (int u = 0; u < SB; ++u)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) eager4(sacc[u][nt], y[nt] + 4 * u);
      if (!full) {
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int t0 = (jg0 + u) * kBlock + 4 * g;
          const bool blk_ok = pb[u] >= 0;  // -1 also for a block past this wavefront's
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[nt][4 * u + i] = (blk_ok && t0 + i <= lim[nt]) ? y[nt][4 * u + i] : -INFINITY;
        }
      }
      if constexpr (!OUT) {
        // Online (max, sum) per lane, one update per stage: the max of the stage's scores first,
        // then the running sum rescaled once by exp2((m_old - m_new) log2 e), which is exactly 1
        // while the max stays (the one-FMA form exp2(m_old log2 e - RN(m_new log2 e)) is off by
        // the product's rounding on every update, and L drifted by ~1e-5 at T = 8192: rel-L2
        // 7e-4 against eager).  A lane sums at most T/32 terms of at most 1 each, so the plain
        // fp32 sum is within ~1e-5 relative of the exact one.  A stage without masked keys has
        // a finite max, and exp2(-inf) = 0 covers the first update.
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float* yt = y[nt];
          static_assert(SB == 4, "the max below covers 16 scores");
          const float m0 = max3f(yt[0], yt[1], yt[2]), m1 = max3f(yt[3], yt[4], yt[5]), m2 = max3f(yt[6], yt[7], yt[8]);
          const float m3 = max3f(yt[9], yt[10], yt[11]), m4 = max3f(yt[12], yt[13], yt[14]);
          const float mt = max3f(max3f(m0, m1, m2), max3f(m3, m4, yt[15]), -INFINITY) * kUnit;
          if (full || mt != -INFINITY) {
#pragma clang fp contract(off)
            const float mn = fmaxf(m_run[nt], mt), nm = -mn * kLog2e;
            const float f = __builtin_amdgcn_exp2f((m_run[nt] - mn) * kLog2e);
            float e[4 * SB];
#pragma unroll
            for (int i = 0; i < 4 * SB; ++i) e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(yt[i], kExpCoef, nm));
            float xs[SB];
#pragma unroll
            for (int u = 0; u < SB; ++u) xs[u] = (e[4 * u] + e[4 * u + 1]) + (e[4 * u + 2] + e[4 * u + 3]);
            l_run[nt] = l_run[nt] * f + ((xs[0] + xs[1]) + (xs[2] + xs[3]));
            m_run[nt] = mn;
          }
        }
      } else {
        // p for each pair h of blocks: the B operand of one p.V product (tokens 4g..4g+3 of the
        // pair's first block, then of its second)
        bf16x8 pop[SB / 2][NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int h = 0; h < SB / 2; ++h) {
            uint32_t pw[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(y[nt][8 * h + 2 * w], kExpCoef, nml[nt]));
              const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(y[nt][8 * h + 2 * w + 1], kExpCoef, nml[nt]));
              pw[w] = pack_bf16x2(p0, p1);
            }
            pop[h][nt] = __builtin_bit_cast(bf16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
          }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int h = 0; h < SB / 2; ++h) {
            const bf16x8 vop = __builtin_bit_cast(bf16x8, sb[(NKC + h * DT + dt) * 64 + lane]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[h][nt], acc[dt][nt], 0, 0, 0);
          }
      }
    };
    fetch(0);
    stash(0);
    fetch(1);
    for (int ss = 0; ss < nst; ++ss) {  // workgroup-uniform
      // stage ss is in LDS for every wavefront, and every wavefront is done with stage ss - 1
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
      stash(ss + 1);  // into the buffer of stage ss - 1
      fetch(ss + 2);
      if (SB * ss < jn) compute_stage(ss, ring[ss & 1]);  // scalar: the stage has keys this wavefront's rows see
    }
  }

  if constexpr (!OUT) {
    // Pass 2's V operand: stage sg of the group (blocks 2sg, 2sg+1) is dequantized by this
    // launch's workgroup sg mod gridDim.x, one dimension tile group per wavefront, as
    // bf16(fp32(code) * scale).  Codes and scales of tokens that are not in the sequence (past
    // T, invalid or absent blocks) become 0, so that no NaN pattern of an unwritten slot reaches
    // the MFMA.
    const int nbk = (T + kBlock - 1) / kBlock;
    for (int sg = (int)blockIdx.x; sg < (nbk + 1) >> 1; sg += (int)gridDim.x) {
      uint32_t w[2][DTW];
      float4 sc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int jb = 2 * sg + u;
        int pb = jb < nbk ? btrow[jb] : -1;
        pb = (pb >= 0 && pb < a.num_blocks) ? pb : -1;
        const int64_t pg = max(pb, 0);
        const uint8_t* vp = vlayer + pg * kpage;
#pragma unroll
        for (int dtl = 0; dtl < DTW; ++dtl) w[u][dtl] = *reinterpret_cast<const uint32_t*>(vp + (voff + dtl * 16u * kBlock));
        sc[u] = *reinterpret_cast<const float4*>(slayer + pg * spage + 4 * g);
        const int t0 = jb * kBlock + 4 * g;
        const int nv = pb >= 0 ? min(max(T - t0, 0), 4) : 0;
        const uint32_t mask = nv >= 4 ? 0xFFFFFFFFu : (1u << (8 * nv)) - 1u;
#pragma unroll
        for (int dtl = 0; dtl < DTW; ++dtl) w[u][dtl] &= mask;
        sc[u].x = nv > 0 ? sc[u].x : 0.0f;
        sc[u].y = nv > 1 ? sc[u].y : 0.0f;
        sc[u].z = nv > 2 ? sc[u].z : 0.0f;
        sc[u].w = nv > 3 ? sc[u].w : 0.0f;
      }
      uint4* dst = a.vhat + ((int64_t)grp * a.vh_stages + sg) * (DT * 64) + lane;
#pragma unroll
      for (int dtl = 0; dtl < DTW; ++dtl) {
        const f32x2 f01 = __builtin_amdgcn_cvt_pk_f32_fp8(w[0][dtl], false);
        const f32x2 f23 = __builtin_amdgcn_cvt_pk_f32_fp8(w[0][dtl], true);
        const f32x2 f45 = __builtin_amdgcn_cvt_pk_f32_fp8(w[1][dtl], false);
        const f32x2 f67 = __builtin_amdgcn_cvt_pk_f32_fp8(w[1][dtl], true);
        dst[(wave * DTW + dtl) * 64] =
            make_uint4(pack_bf16x2(f01.x * sc[0].x, f01.y * sc[0].y), pack_bf16x2(f23.x * sc[0].z, f23.y * sc[0].w),
                       pack_bf16x2(f45.x * sc[1].x, f45.y * sc[1].y), pack_bf16x2(f67.x * sc[1].z, f67.y * sc[1].w));
      }
    }
  }

  if constexpr (!OUT) {
    // (max, sum) of each row over the four lane groups, in a fixed order
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float m = m_run[nt], l = l_run[nt];
      merge_lanes<16>(m, l);
      merge_lanes<32>(m, l);
      if (g == 0 && rv[nt]) st[(int64_t)(row0 + nt * 16 + n) * a.pf_split + split] = make_float2(m, l);
    }
  } else {
    // lane (g, n) holds O^T[dims dt*16 + 4g .. +3][row nt*16 + n] of this part's keys
    bool write = true;
    if (nparts > 1) {  // workgroup-uniform
      // Every part writes its fp32 partial to its slot (device-scope stores), waits for them,
      // and counts itself in the row group's counter -- a (call tag, count) word in the sync
      // area, read as 0 when it carries another call's tag.  The part that completes the count
      // sums the slots in part order (its own from registers), writes the output and zeroes the
      // counter.  Nobody waits for anybody: the order of arrival changes who sums, not the sum.
      const int nrg = (a.R + kPass2Rows - 1) / kPass2Rows;
      constexpr int slot_b = kPass2Rows * D * 4;  // bytes per part slot
      // the row group's slots, written and read with 16-byte device-scope (sc1) accesses
      const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
          a.partial + ((int64_t)grp * nrg + rgi) * a.pf_parts * (slot_b / 4), (short)0, nparts * slot_b, 0x00020000);
      // lane (g, n): row wave*ROWS + nt*16 + n, dimensions dt*16 + 4g .. +3
      const int lofs = ((wave * ROWS + n) * D + 4 * g) * 4;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[dt][nt]), srs,
                                                 split * slot_b + lofs + (nt * 16 * D + dt * 16) * 4, 0, 16);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      SDV_VMCNT0();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __syncthreads();
      __shared__ int s_last;
      if (tid == 0) {
        uint64_t* ctr = reinterpret_cast<uint64_t*>(a.sync) + kSyncHeadBytes / 8 + (int64_t)grp * nrg + rgi;
        uint64_t old = load_dev_u64(ctr);
        uint32_t mine = 0;
        for (;;) {  // compare-and-swap against the other parts of this row group only
          const uint32_t cnt = (uint32_t)(old >> 32) == a.tag ? (uint32_t)old : 0u;
          const uint64_t nw = ((uint64_t)a.tag << 32) | (cnt + 1u);
          const uint64_t prev = atomicCAS(reinterpret_cast<unsigned long long*>(ctr), (unsigned long long)old,
                                          (unsigned long long)nw);
          if (prev == old) {
            mine = cnt + 1u;
            break;
          }
          old = prev;
        }
        const bool last = mine == (uint32_t)nparts;
        if (last) store_dev_u64(ctr, 0);
        s_last = last;
      }
      __syncthreads();
      write = s_last;
      if (write) {
        // the parts' sum in part order, each part's slot loaded whole before it is added
        f32x4 sum[DT][NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) sum[dt][nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < nparts; ++k) {  // workgroup-uniform
          f32x4 v[DT][NT];
          if (k == split) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
              for (int dt = 0; dt < DT; ++dt) v[dt][nt] = acc[dt][nt];
          } else {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
              for (int dt = 0; dt < DT; ++dt)
                v[dt][nt] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, k * slot_b + lofs + (nt * 16 * D + dt * 16) * 4, 0, 16));
          }
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) sum[dt][nt] += v[dt][nt];
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt][nt] = sum[dt][nt];
      }
    }
    if (write) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if (!rv[nt]) continue;
        const int r = row0 + nt * 16 + n, hl = r / a.S, si = r % a.S;
        uint16_t* op = a.out + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          *reinterpret_cast<uint2*>(op + dt * 16) =
              make_uint2(pack_bf16x2(acc[dt][nt][0], acc[dt][nt][1]), pack_bf16x2(acc[dt][nt][2], acc[dt][nt][3]));
      }
    }
  }
}

// ---------------------------------------------------------------------------- group
// Many (layer*batch, KV head) groups of one row tile each -- decode and short verify over many
// sequences (config 4: 28 layers x 32 ragged sequences x 2 KV heads = 1792 groups) -- in one
// launch of persistent workgroups, one per CU, that take whole groups from a claim counter in
// the order of decreasing sequence length (the long groups first, the short ones last, so the
// workgroups finish together).  A group is done by one workgroup alone and no workgroup ever
// waits for another:
//   1. q.k^T: wavefront w takes blocks w, w+W, ... (two in flight); the BF16 scores of row n go
//      to the workgroup's own scratch rows in the workspace, and
//      each wavefront keeps a running (max, sum) per row, rescaled exactly (factor 1 while the
//      max stays).
//   2. The wavefronts' pairs are merged in wavefront order in LDS: (M, 1/L) per row.
//   3. p.V: wavefront w takes stages of 4 blocks w, w+W, ... (lane group g: block 4*stage + g),
//      p = bf16(exp(s - M) / L) from the scratch scores, V dequantized in registers, O^T on the
//      MFMA (pv_compute, as in the three-launch p.V kernel); the wavefronts' outputs are summed in
//      wavefront order in LDS and stored as BF16.
// Every reduction has a fixed order, so results do not depend on which workgroup took which
// group.  Words 2 and 3 of the synchronisation area hold the claim counter and the count of
// finished workgroups; the last workgroup to finish zeroes both for the next call.
constexpr int kGroupWaves = 8;
constexpr int kGroupGrid = 256;          // workgroups (one per CU of the MI355X)
constexpr int kGroupMaxBlocks = 4096;    // page ids of one group staged in LDS: T <= 65536
constexpr int kGroupSortMax = 1024;      // batches up to this size are ordered by length
// Fewest groups this kernel takes: one per workgroup.  Between that and the 1,024 groups it
// once started at (one-tile groups the single launch cannot hold at once, with too little work
// per layer for one single launch per layer), it beats the three launches on every shape
// measured: one layer of 160 ragged sequences up to 3K tokens 63.1 -> 50.8 us, 300 x 2K
// 112 -> 108 us, 480 ragged up to 4K 214.6 -> 181.9 us, 2 layers x 200 x 1K 85.5 -> 77.0 us.
constexpr int kGroupMinGroups = kGroupGrid;
// K blocks and V stages (4 blocks) in flight per wavefront.  Deeper rings measured no faster on
// config 4 (K 3-4, V 3: 2.55-2.60 ms against 2.54 ms)
constexpr int kGroupKRing = 2;
constexpr int kGroupVRing = 2;
static_assert(kGroupSortMax <= kGroupMaxBlocks, "the lengths are staged in the page-id array");

template <int D>
__global__ __launch_bounds__(64 * kGroupWaves) void group_kernel(AttnArgs a, int n_groups, int layers, int tpad) {
  constexpr int W = kGroupWaves, NTHR = 64 * W, KK = D / 32, DT = D / 16;
  __shared__ int s_order[kGroupSortMax];
  __shared__ int lpb[kGroupMaxBlocks];
  __shared__ float2 lst[W][16];
  __shared__ float2 lgs[16];
  __shared__ float lacc[W][16][D + 4];  // +4: spread the lane groups over LDS banks
  __shared__ int s_claim;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int per_seq = layers * a.KV;
  const bool sorted = a.B <= kGroupSortMax;
  if (sorted) {  // s_order[rank] = sequence: decreasing length, lower index first on ties
    int* s_len = lpb;  // the lengths, staged in the page-id array before its first use
    for (int b = tid; b < a.B; b += NTHR) s_len[b] = seq_len_of(a, b);
    __syncthreads();
    for (int b = tid; b < a.B; b += NTHR) {
      const int tb = s_len[b];
      int rank = 0;
      for (int c = 0; c < a.B; ++c) {
        const int tc = s_len[c];
        rank += (tc > tb) || (tc == tb && c < b);
      }
      s_order[rank] = b;
    }
  }
  uint16_t* scr = a.scores + (int64_t)blockIdx.x * a.R * tpad;  // this workgroup's score rows
  const int prow = n < a.R ? n : 0;  // row this lane's probabilities come from (padding: row 0)
#ifdef SDV_PHASE_TRACE
  if (tid == 0 && blockIdx.x < kPhaseTraceGroups)
    for (int w = 10; w < 14; ++w) phase_trace[blockIdx.x * kPhaseSlots + w] = 0;
#endif
  unsigned long long t0 = SDV_CLOCK();
  for (;;) {
    __syncthreads();  // the previous group's LDS reads are done (and s_order is written)
    if (tid == 0) s_claim = (int)atomicAdd(a.sync + 2, 1u);
    __syncthreads();
    const int k = s_claim;
    if (k >= n_groups) break;
    const int rk = k / per_seq, rem = k - rk * per_seq;
    const int layer = rem / a.KV, kvh = rem - layer * a.KV;
    const int b = sorted ? s_order[rk] : rk;
    const int T = seq_len_of(a, b);
    const int nblk = (T + kBlock - 1) >> 4;

    // q rows: lane (g, n) holds row n, dimensions kk*32 + 8g .. +7 (the B operand of S^T = K Q^T)
    bf16x8 qop[KK];
    int lim;  // last key row n sees
    {
      const bool rv = n < a.R;
      const int hl = rv ? n / a.S : 0, si = rv ? n % a.S : 0;
      const uint16_t* qp = a.q + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + g * 8;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) qop[kk] = rv ? load_bf16x8(qp + kk * 32) : zero_bf16x8();
      lim = T - a.S + si;
    }
    const int* btrow = a.block_table + (int64_t)b * a.max_blocks;
    for (int j = tid; j < nblk; j += NTHR) {
      const int pb = btrow[j];
      lpb[j] = (pb >= 0 && pb < a.num_blocks) ? pb : -1;
    }
    __syncthreads();
    unsigned long long t1 = SDV_CLOCK();
    SDV_PHASE_ADD(10, t1 - t0);

    // ------------------------------------------------------------------ 1. q.k^T
    float m_run = -INFINITY, l_run = 0.0f;  // row n; identical in the four lane groups
    {
      const uint16_t* kbase = a.k_pages + layer * a.k_ls + (int64_t)lane * 8;
      // a block past the group reads block 0 (the wait counters stay exact) and is not computed
      auto kload = [&](int j, bf16x8 (&kop)[KK], int& pb) {
        pb = j < nblk ? lpb[j] : -1;
        const uint16_t* kp = kbase + ((int64_t)max(pb, 0) * a.KV + kvh) * (kBlock * D);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) kop[kk] = __builtin_bit_cast(bf16x8, load_stream16(kp + kk * 512));
      };
      auto kcompute = [&](const bf16x8 (&kop)[KK], int pb, int j) {
        f32x4 acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[kk], qop[kk], acc, 0, 0, 0);
        const int tb = j * kBlock + 4 * g;  // this lane's first token
        float s4[4];
        float mt = -INFINITY;
        float y[4];
        round_scaled4(acc[0], acc[1], acc[2], acc[3], a.inv_sqrt_d, y);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = y[i];
          s4[i] = (pb >= 0 && tb + i <= lim) ? x : -INFINITY;
          mt = fmaxf(mt, s4[i]);
        }
        if (n < a.R)
          *reinterpret_cast<uint2*>(scr + (int64_t)n * tpad + tb) =
              make_uint2(pack_bf16x2(s4[0], s4[1]), pack_bf16x2(s4[2], s4[3]));
        // the block's (max, sum) of row n over the four lane groups, then the running pair
        float2 pm = lane_pair<16>(mt);
        float M = fmaxf(pm.x, pm.y);
        pm = lane_pair<32>(M);
        M = fmaxf(pm.x, pm.y);
        const float nml = M == -INFINITY ? 0.0f : -M * kLog2e;  // empty block: every exp is 0
        float l = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) l += __builtin_amdgcn_exp2f(__builtin_fmaf(s4[i], kLog2e, nml));
        float2 pl = lane_pair<16>(l);
        l = pl.x + pl.y;
        pl = lane_pair<32>(l);
        l = pl.x + pl.y;
        const float mn = fmaxf(m_run, M);
        const float f_old = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - mn) * kLog2e);
        const float f_new = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((M - mn) * kLog2e);
        l_run = l_run * f_old + l * f_new;
        m_run = mn;
      };
      // a ring of kGroupKRing blocks in flight; one loop exit, at the head, and every buffer
      // reloaded (kGroupKRing * W blocks ahead) right after it is used
      bf16x8 kr[kGroupKRing][KK];
      int pr[kGroupKRing];
#pragma unroll
      for (int i = 0; i < kGroupKRing; ++i) kload(wave + i * W, kr[i], pr[i]);
      for (int j = wave; j < nblk; j += kGroupKRing * W) {
#pragma unroll
        for (int i = 0; i < kGroupKRing; ++i) {
          const int jj = j + i * W;
          if (jj < nblk) kcompute(kr[i], pr[i], jj);  // wave-uniform
          kload(jj + kGroupKRing * W, kr[i], pr[i]);
        }
      }
    }
    if (g == 0) lst[wave][n] = make_float2(m_run, l_run);
    __syncthreads();  // also makes the scratch scores visible to the whole workgroup

    // ------------------------------------------------------------------ 2. (M, 1/L) per row
    if (tid < 16) {
      float m = lst[0][tid].x, l = lst[0][tid].y;
#pragma unroll
      for (int w = 1; w < W; ++w) merge_fast(m, l, lst[w][tid].x, lst[w][tid].y);
      lgs[tid] = make_float2(m, 1.0f / l);
    }
    __syncthreads();
    t0 = SDV_CLOCK();
    SDV_PHASE_ADD(11, t0 - t1);

    // ------------------------------------------------------------------ 3. p.V
    float gm[1], ginv[1];
    gm[0] = lgs[prow].x;
    ginv[0] = lgs[prow].y;
    f32x4 acc[DT][1];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt][0] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    {
      const uint8_t* vlayer = a.v_pages + layer * a.v_ls;
      const float* slayer = a.v_scales + layer * a.s_ls;
      const uint16_t* srow_p = scr + (int64_t)prow * tpad;
      const int nst = (nblk + 3) >> 2;
      const int full_blocks = T >> 4;
      // lane group g takes block 4*st + g; a block past the group reads block 0 and the first
      // block's scores, and is sanitized (no token) when its stage is computed
      auto vload = [&](int st_i, PvStage<D, 1>& x) {
        const int jb = 4 * st_i + g;
        const int pb = jb < nblk ? lpb[jb] : -1;
        x.ok = pb >= 0;
        x.blk = jb;
        const int64_t page = (int64_t)(x.ok ? pb : 0) * a.KV + kvh;
        const uint8_t* vp = vlayer + (page * D + n) * kBlock;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) x.code[dt] = load_stream16(vp + dt * 16 * kBlock);
        x.scl = __builtin_nontemporal_load(slayer + page * kBlock + n);
        const uint4* ps = reinterpret_cast<const uint4*>(srow_p + (int64_t)(jb < nblk ? jb : 0) * kBlock);
        x.sc[0][0] = ps[0];
        x.sc[0][1] = ps[1];
      };
      PvStage<D, 1> vr[kGroupVRing];
#pragma unroll
      for (int i = 0; i < kGroupVRing; ++i) vload(wave + i * W, vr[i]);
      for (int st_i = wave; st_i < nst; st_i += kGroupVRing * W) {
#pragma unroll
        for (int i = 0; i < kGroupVRing; ++i) {
          const int ss = st_i + i * W;
          if (ss < nst) pv_compute<D, 1>(vr[i], acc, gm, ginv, T, 4 * ss + 3 < full_blocks, n);  // wave-uniform
          vload(ss + kGroupVRing * W, vr[i]);
        }
      }
    }
    // lane (g, n) holds O^T[dims dt*16 + 4g .. +3][row n]; the wavefronts are summed in order
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) lacc[wave][n][dt * 16 + 4 * g + i] = acc[dt][0][i];
    __syncthreads();
    for (int e = tid; e * 4 < a.R * D; e += NTHR) {
      const int r = (4 * e) / D, d = 4 * e - r * D;
      float4 sm = *reinterpret_cast<const float4*>(&lacc[0][r][d]);
#pragma unroll
      for (int w = 1; w < W; ++w) {
        const float4 f = *reinterpret_cast<const float4*>(&lacc[w][r][d]);
        sm.x += f.x; sm.y += f.y; sm.z += f.z; sm.w += f.w;
      }
      const int hl = r / a.S, si = r % a.S;
      uint16_t* dst = a.out + layer * a.q_ls + b * a.q_sb + (int64_t)(kvh * a.G + hl) * a.q_sh + si * a.q_ss + d;
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(sm.x, sm.y), pack_bf16x2(sm.z, sm.w));
    }
    t1 = SDV_CLOCK();
    SDV_PHASE_ADD(12, t1 - t0);
    SDV_PHASE_ADD(13, 1ull);
    t0 = t1;
  }
  // the last workgroup to finish leaves the counters zero for the next call
  if (tid == 0 && atomicAdd(a.sync + 3, 1u) == gridDim.x - 1) {
    __hip_atomic_store(a.sync + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.sync + 3, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------- planning
struct Plan {
  int NT, n_row_groups, rpad;
  int qk_bpw, qk_chunk_tokens, n_qk_chunks;
  int pv_bpw, pv_chunk_tokens, n_pv_chunks;
  int score_stride;
  size_t off_scores, off_stats, off_partial;     // three-launch layout (after the sync area)
  int64_t groups;
  bool group;                                     // group_kernel serves the call (many one-tile groups)
  int tpad;                                       // group_kernel: scratch row length (tokens)
  int pf_parts;                                   // prefill pass 2: key parts per row group
  int pf_split;                                   // prefill pass 1: key parts per row group
  int pf_kstar, pf_wh;                            // prefill pass 2: parts by key count (0: uniform)
  size_t off_vhat;                                // prefill: dequantized V (pass 1 -> pass 2)
  int vh_stages;                                  // prefill: two-block stages per group
  size_t total;                                   // bytes for every layout the call may take
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
  // then streams its blocks through the load pipeline.  Large problems give pv wavefronts
  // up to 64 blocks (measured on config 4, B=32 x 28 layers: p.V 1187 us at 32 -> 1037 us at
  // 64); 64 is also the most pv_kernel can take: it holds one page id per lane.
  int qb = 1;
  const int qb_max = kQkScoreTokens / (kBlock * p->NT) >= 1 ? kQkScoreTokens / (kBlock * p->NT) : 1;
  while (qb < qb_max && blocks > (int64_t)kWaves * qb * 1024) qb *= 2;
  int pb = 4;  // multiple of the 4-block pv stage
  while (pb < kWave && blocks > (int64_t)kWaves * pb * 512) pb *= 2;
  p->qk_bpw = qb;
  p->qk_chunk_tokens = kWaves * qb * kBlock;
  p->n_qk_chunks = (max_seq_len + p->qk_chunk_tokens - 1) / p->qk_chunk_tokens;
  p->pv_bpw = pb;
  p->pv_chunk_tokens = kWaves * pb * kBlock;
  p->n_pv_chunks = (max_seq_len + p->pv_chunk_tokens - 1) / p->pv_chunk_tokens;
  p->score_stride = max(p->n_qk_chunks * p->qk_chunk_tokens, p->n_pv_chunks * p->pv_chunk_tokens);
  const int64_t groups = (int64_t)L * B * KV;
  p->groups = groups;
  p->group = false;
  p->tpad = 0;
  p->pf_parts = 1;
  p->pf_split = 1;
  p->pf_kstar = 0;
  p->pf_wh = 0;
  p->off_vhat = 0;
  p->vh_stages = 0;
  if (p->n_row_groups > 1) {  // prefill kernels: the per-row (max, sum) of each key part
    p->off_scores = kSyncBytes;
    p->off_stats = kSyncBytes;
    const int nbk = (max_seq_len + kBlock - 1) / kBlock;
    const int max_parts = min(kPrefillMaxParts, max(1, nbk / 8));
    const int64_t nrg1 = (R + kPass1Tiles * kPrefillRows * kPass1Waves - 1) / (kPass1Tiles * kPrefillRows * kPass1Waves);
    p->pf_split = (int)std::max<int64_t>(1, std::min<int64_t>(max_parts, pass1_workgroups(D) / (groups * nrg1)));
    const size_t stats = round_up((size_t)(groups * R * 8 * p->pf_split), 256);
    p->off_partial = p->off_stats + stats;
    // pass 2 splits the keys too when its counters (one per row group) fit the sync area's
    // statistics region; its part slots follow the statistics
    const int64_t nrg = (R + kPass2Rows - 1) / kPass2Rows;
    p->pf_parts = groups * nrg <= (int64_t)(kSyncStatsBytes / 8)
                      ? (int)std::max<int64_t>(1, std::min<int64_t>(std::min(max_parts, kPrefillMaxParts2), pass2_workgroups(D) / (groups * nrg)))
                      : 1;
    // With S a multiple of the pass's rows, the parts of each row group follow its key count
    // (the offset-causal mask: the head's later rows see more keys): the fewest blocks per
    // part that keep the launch within the same budget, so that the workgroups carry nearly
    // equal work (2048 x 8192, 12/2/128: 504 workgroups of at most 216 blocks instead of 384 of
    // up to 256, half of the CUs holding one)
    p->pf_kstar = 0;
    p->pf_wh = 0;
    if (p->pf_parts > 1 && S % kPass2Rows == 0) {
      const int rgph = S / kPass2Rows;
      const int64_t heads = groups * G;  // (layer, sequence, query head): rgph row groups each
      for (int kstar = kStageBlocks; kstar < nbk + kStageBlocks; kstar += kStageBlocks) {
        int wh = 0, pmax = 0;
        for (int k = 0; k < rgph; ++k) {
          const int pk = pass2_group_parts(k, S, max_seq_len, kPass2Rows, kstar);
          wh += pk;
          pmax = std::max(pmax, pk);
        }
        if (heads * wh <= pass2_workgroups(D) && pmax <= kPrefillMaxParts2) {
          if (pmax > 1) {
            p->pf_kstar = kstar;
            p->pf_wh = wh;
            p->pf_parts = pmax;
          }
          break;
        }
      }
    }
    const size_t parts = p->pf_parts > 1
                             ? round_up((size_t)(groups * nrg * p->pf_parts * kPass2Rows * D * 4), 256)
                             : 0;
    // pass 1 dequantizes V once for pass 2: D/16 x 1 KiB per stage of two blocks
    p->vh_stages = (((max_seq_len + kBlock - 1) / kBlock) + 1) / 2;
    p->off_vhat = p->off_partial + parts;
    p->total = p->off_vhat + (size_t)groups * p->vh_stages * (D / 16) * 1024;
    return true;
  }
  // the sync area [0, kSyncBytes) is shared by every layout and only the fused kernel uses it
  const size_t scores = round_up((size_t)(groups * R * p->score_stride * 2), 256);
  const size_t stats = round_up((size_t)(groups * p->n_qk_chunks * p->rpad * 8), 256);
  const size_t partial = round_up((size_t)(groups * p->n_pv_chunks * R * D * 4), 256);
  p->off_scores = kSyncBytes;
  p->off_stats = p->off_scores + scores;
  p->off_partial = p->off_stats + stats;
  // the fused kernel keeps its statistics and partials inside the sync area
  p->total = p->off_partial + partial;
  // group_kernel: words 2-3 of the sync area, then R score rows per workgroup at off_scores
  // (the profiling split refuses these shapes, so the three-launch layout is not needed)
  p->group = p->NT == 1 && groups >= kGroupMinGroups && max_seq_len <= kGroupMaxBlocks * kBlock;
  p->tpad = p->group ? (int)round_up((size_t)max_seq_len, kBlock) : 0;
  if (p->group) p->total = kSyncBytes + round_up((size_t)kGroupGrid * R * p->tpad * 2, 256);
  return true;
}

// Resident workgroup capacity of fused_kernel<D, NT> with `lds` bytes of dynamic LDS on the
// current device (cached per device and 4 KiB LDS bucket); 0 when the device cannot run it.
// Above 64 KiB of dynamic LDS the kernel's limit is raised first (once per device and size).
template <int D, int NT, int W, int NTG>
static int fused_capacity(size_t lds) {
  constexpr int kBuckets = 41;  // 0 .. 160 KiB
  static std::atomic<int> cache[64][kBuckets];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int bucket = (int)((lds + 4095) / 4096);
  if (bucket >= kBuckets) return 0;
  int cap = cache[dev][bucket].load(std::memory_order_relaxed);
  if (cap > 0) return cap;
  if ((size_t)bucket * 4096 > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(fused_kernel<D, NT, W, NTG>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, bucket * 4096) != hipSuccess) {
    (void)hipGetLastError();  // leave no error behind for the launch status check
    return 0;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fused_kernel<D, NT, W, NTG>, 64 * W,
                                                   (size_t)bucket * 4096) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  per_cu = min(per_cu, fused_max_per_cu<D, NT>());
  cap = per_cu * cus;
  cache[dev][bucket].store(cap, std::memory_order_relaxed);
  return cap;
}

struct FusedShape {
  int gb, base, layers, maxblk, grid, ntg;
  size_t lds;
};

// The single-launch shape: as many workgroups as the device holds at once (at most
// kFusedGroupItems items per group, items of at least one page block), or false when another
// path must serve the call (several query-row groups, more groups than the device holds at
// once, items too large for LDS).  per_seq_layers > 0: a batch of 2..64 sequences with
// per-sequence lengths over that many layers, whose items the kernel sizes per sequence.
template <int D, int NT, int W>
static bool fused_shape(const Plan& p, int R, int max_seq_len, int per_seq_layers, FusedShape* f) {
  if (p.n_row_groups != 1 || p.groups > kFusedMaxItems) return false;
  const int G = (int)p.groups;
  const int gb = (max_seq_len + kBlock - 1) / kBlock;
  // at most kFusedGroupItems items of at least one block: a small problem (one layer) spread
  // over every CU would spend its time in the cross-workgroup exchanges
  const int max_items = min(kFusedGroupItems, gb);
  // items whose fp32 partials fit the sync area
  const int part_cap = (int)(kSyncPartBytes / ((size_t)R * D * 4));
  constexpr int NTGN = fused_ntg(D, W), NTGW = fused_ntg_wide(D, W, NT);
  int cap = min(part_cap, fused_capacity<D, NT, W, NTGN>((size_t)fused_lds_layout(R, D, 1, W, NT == 1, NTGN).total));
  for (int iter = 0; iter < 4; ++iter) {
    if (cap < G) return false;
    const int base = min(max_items, cap / G);
    const int maxblk = (gb + base - 1) / base;
    const int ntg = maxblk >= kWideMinBlocks ? NTGW : NTGN;
    const size_t lds = (size_t)fused_lds_layout(R, D, maxblk, W, NT == 1, ntg).total;
    if (lds > 160 * 1024) return false;
    const int cap2 =
        min(part_cap, ntg == NTGN ? fused_capacity<D, NT, W, NTGN>(lds) : fused_capacity<D, NT, W, NTGW>(lds));
    if (cap2 < cap) {  // a wider item needs more LDS: the device holds fewer of them
      cap = cap2;
      continue;
    }
    // Groups of one length (one sequence, or no per-sequence lengths) get the same number of
    // items each, even if some CUs stay idle: extra items would only shrink the items of some
    // groups, while the largest items set the end of the call, and the workgroups left with
    // them stream alone at the end (28 layers at 8K: 224 equal items 39.4 us against 256 mixed
    // items of 102 and 128 blocks 41.2 us).  A batch with per-sequence lengths launches every
    // workgroup the device holds and the kernel gives each sequence items in proportion to its
    // length, none over maxblk blocks (a config-4 layer, 32 sequences of 2K-32K tokens: the
    // longest groups' 512-block items became about 340 blocks).
    const int grid = per_seq_layers > 0 ? cap : G * base;
    if (grid > kFusedMaxItems || grid > part_cap) return false;
    f->gb = gb;
    f->base = base;
    f->layers = per_seq_layers;
    f->maxblk = maxblk;
    f->grid = grid;
    f->ntg = ntg;
    f->lds = lds;
    return true;
  }
  return false;
}

template <int D, int NT, int W>
static bool try_fused_w(AttnArgs a, const Plan& p, hipStream_t st) {
  FusedShape f;
  const int psl = (a.seq_lens && a.B > 1 && a.B <= kWave) ? (int)(p.groups / ((int64_t)a.B * a.KV)) : 0;
  if (!fused_shape<D, NT, W>(p, a.R, a.max_seq_len, psl, &f)) return false;
  a.f_gb = f.gb;
  a.f_base = f.base;
  a.f_layers = f.layers;
  a.f_maxblk = f.maxblk;
  constexpr int NTGN = fused_ntg(D, W), NTGW = fused_ntg_wide(D, W, NT);
  if (f.ntg == NTGN)
    hipLaunchKernelGGL((fused_kernel<D, NT, W, NTGN>), dim3((unsigned)f.grid), dim3(64 * W), f.lds, st, a);
  else
    hipLaunchKernelGGL((fused_kernel<D, NT, W, NTGW>), dim3((unsigned)f.grid), dim3(64 * W), f.lds, st, a);
  return true;
}

// One row tile with an in-kernel append runs 16 wavefronts: the draft chain (D=64, 5 steps x 24
// layers at 8K, append + attention per layer) takes 1275 us with 16 against 1343 us with 8,
// and 5 x 28 D=128 decode steps 1710 against 1735 us, while the same calls without the append
// are faster with 8 (draft chain in two launches per layer: 1601 -> 1551 us).  Two row tiles
// keep 8 (the 28-layer verify step with its appends: 441 us, 493 us with 16).
template <int D, int NT>
static bool try_fused(AttnArgs a, const Plan& p, hipStream_t st) {
  if constexpr (NT == 1)
    if (a.app_v) return try_fused_w<D, NT, 16>(a, p, st);
  return try_fused_w<D, NT, fused_waves<D, NT>()>(a, p, st);
}

// workgroups of the single-launch kernel for these sizes, or 0 (another path); per_seq_layers
// as for fused_shape (whether the single launch serves a shape does not depend on it).
// append: the call writes new tokens in the kernel, which try_fused launches with the
// wavefront count of an appending call (more LDS for one row tile, so a shape may fit without
// the append and not with it): the answer is the one try_fused will act on.
template <int D>
static int fused_grid_for(const Plan& p, int R, int max_seq_len, int per_seq_layers = 0, bool append = false) {
  FusedShape f;
  bool ok = false;
  switch (p.NT) {
    case 1:
      ok = append ? fused_shape<D, 1, 16>(p, R, max_seq_len, per_seq_layers, &f)
                  : fused_shape<D, 1, fused_waves<D, 1>()>(p, R, max_seq_len, per_seq_layers, &f);
      break;
    case 2: ok = fused_shape<D, 2, fused_waves<D, 2>()>(p, R, max_seq_len, per_seq_layers, &f); break;
    case 3: ok = fused_shape<D, 3, fused_waves<D, 3>()>(p, R, max_seq_len, per_seq_layers, &f); break;
    default: ok = fused_shape<D, 4, fused_waves<D, 4>()>(p, R, max_seq_len, per_seq_layers, &f); break;
  }
  return ok ? f.grid : 0;
}

template <int D, int NT>
static void launch_qk_pv(const AttnArgs& a, const Plan& p, int zdim, hipStream_t st, int phases) {
  const unsigned gy = a.KV * p.n_row_groups;
  if (phases & SDV_PHASE_QK)
    hipLaunchKernelGGL((qk_kernel<D, NT>), dim3(p.n_qk_chunks, gy, zdim), dim3(256), 0, st, a);
  if (phases & SDV_PHASE_PV)
    hipLaunchKernelGGL((pv_kernel<D, NT>), dim3(p.n_pv_chunks, gy, zdim), dim3(256), 0, st, a);
}

// Tag of a single-launch call: unique among the process's calls (never 0; 31 bits), with
// kTagGraph set when the stream is recording a graph (whose replays reuse the tag).
static std::atomic<uint32_t> g_calls{0};
static std::atomic<uint32_t> g_wait_limit{0};  // 0: kDefaultSpinLimit

static uint32_t next_call_tag(hipStream_t st) {
  uint32_t t = 0;
  while (t == 0) t = (g_calls.fetch_add(1, std::memory_order_relaxed) + 1u) & ~kTagGraph;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess)
    (void)hipGetLastError();
  else if (cs == hipStreamCaptureStatusActive)
    t |= kTagGraph;
  return t;
}

// polls per wait for the kernels: 0 (from UINT32_MAX) makes every wait give up at its first
// check, published or not (tests of the failure path)
static uint32_t wait_limit() {
  const uint32_t v = g_wait_limit.load(std::memory_order_relaxed);
  return v == 0xFFFFFFFFu ? 0u : v ? v : kDefaultSpinLimit;
}

// A multi-layer problem the single launch cannot hold at once, whose layers it can, with at least
// this much work per layer (batch x KV heads x max_seq_len): one single launch per layer on the
// same stream, each with its own call tag.  A config-4 call (28 layers x 32 sequences of 2K-32K
// tokens) takes 28 x 85 us this way against 2.57 ms on the per-group kernel; with little work
// per layer the per-group kernel's one launch wins (a one-layer call costs about 9 us).
constexpr int64_t kPerLayerMinWork = 1 << 18;

template <int D>
static bool try_fused_per_layer(const AttnArgs& a, int layers, hipStream_t st) {
  if (layers < 2 || (int64_t)a.B * a.KV * a.max_seq_len < kPerLayerMinWork) return false;
  Plan pl;
  if (!make_plan(1, a.B, a.G * a.KV, a.KV, a.S, D, a.max_seq_len, &pl) || pl.n_row_groups != 1 ||
      fused_grid_for<D>(pl, a.R, a.max_seq_len) <= 0)
    return false;
  for (int l = 0; l < layers; ++l) {
    AttnArgs al = a;
    al.q = a.q + l * a.q_ls;
    al.out = a.out + l * a.q_ls;
    al.k_pages = a.k_pages + l * a.k_ls;
    al.v_pages = a.v_pages + l * a.v_ls;
    al.v_scales = a.v_scales + l * a.s_ls;
    al.k_ls = al.v_ls = al.s_ls = 0;
    al.q_ls = 0;
    if (l > 0) al.tag = next_call_tag(st);
    switch (pl.NT) {
      case 1: try_fused<D, 1>(al, pl, st); break;
      case 2: try_fused<D, 2>(al, pl, st); break;
      case 3: try_fused<D, 3>(al, pl, st); break;
      default: try_fused<D, 4>(al, pl, st); break;
    }
  }
  return true;
}

// Launches the call's kernels.  Only the single launch writes new tokens itself: a call with
// a.app_v set that the single launch does not take returns false before anything is launched,
// and the caller appends with the append kernel and calls again without a.app_v.
template <int D>
static bool launch_all(const AttnArgs& a, const Plan& p, int zdim, hipStream_t st, int phases) {
  if (p.n_row_groups > 1) {  // many query rows: the two prefill passes
    if (a.app_v) return false;
    const dim3 grid((unsigned)((a.R + kPass2Rows - 1) / kPass2Rows), a.KV, zdim);
    constexpr int rows1 = kPass1Tiles * 16 * kPass1Waves;  // pass 1 rows per workgroup
    const dim3 grid1((unsigned)((a.R + rows1 - 1) / rows1) * a.pf_split, grid.y, grid.z),
        grid2(a.pf_kstar > 0 ? (unsigned)(a.G * a.pf_wh) : grid.x * a.pf_parts, grid.y, grid.z);
    if (phases & SDV_PHASE_QK) hipLaunchKernelGGL((prefill_kernel<D, false>), grid1, dim3(64 * kPass1Waves), 0, st, a);
    if (phases & SDV_PHASE_PV) hipLaunchKernelGGL((prefill_kernel<D, true>), grid2, dim3(64 * kPass2Waves), 0, st, a);
    return true;
  }
  if (phases == SDV_PHASE_ALL) {
    bool done = false;
    switch (p.NT) {
      case 1: done = try_fused<D, 1>(a, p, st); break;
      case 2: done = try_fused<D, 2>(a, p, st); break;
      case 3: done = try_fused<D, 3>(a, p, st); break;
      default: done = try_fused<D, 4>(a, p, st); break;
    }
    if (done) return true;
    if (a.app_v) return false;
    if (try_fused_per_layer<D>(a, zdim / a.B, st)) return true;
    if (p.group) {  // many one-tile groups: persistent workgroups, whole groups each
      hipLaunchKernelGGL(group_kernel<D>, dim3(kGroupGrid), dim3(64 * kGroupWaves), 0, st, a, (int)p.groups,
                         zdim / a.B, p.tpad);
      return true;
    }
  }
  if (a.app_v) return false;
  switch (p.NT) {
    case 1: launch_qk_pv<D, 1>(a, p, zdim, st, phases); break;
    case 2: launch_qk_pv<D, 2>(a, p, zdim, st, phases); break;
    case 3: launch_qk_pv<D, 3>(a, p, zdim, st, phases); break;
    default: launch_qk_pv<D, 4>(a, p, zdim, st, phases); break;
  }
  if (phases & SDV_PHASE_REDUCE)
    hipLaunchKernelGGL(reduce_kernel<D>, dim3((a.R * D + 63) / 64, a.KV, zdim), dim3(256), 0, st, a);
  return true;
}

// Workspace bytes the path launch_all takes for a call touches: the synchronisation area for
// the single launch (also one per layer), the full layout otherwise (per-group kernel, three
// launches, prefill rows).  The same decisions as launch_all and try_fused_per_layer.
template <int D>
static size_t path_workspace(const Plan& p, const AttnArgs& a, int layers, bool append) {
  if (p.n_row_groups > 1) return p.total;
  const int psl = (a.seq_lens && a.B > 1 && a.B <= kWave) ? layers : 0;
  if (fused_grid_for<D>(p, a.R, a.max_seq_len, psl, append) > 0) return kSyncBytes;
  // otherwise the append kernel runs first and the call takes the path of a call without it
  if (append && fused_grid_for<D>(p, a.R, a.max_seq_len, psl) > 0) return kSyncBytes;
  if (layers >= 2 && (int64_t)a.B * a.KV * a.max_seq_len >= kPerLayerMinWork) {
    Plan pl;
    if (make_plan(1, a.B, a.G * a.KV, a.KV, a.S, D, a.max_seq_len, &pl) && pl.n_row_groups == 1 &&
        fused_grid_for<D>(pl, a.R, a.max_seq_len) > 0)
      return kSyncBytes;
  }
  return p.total;
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

// The new tokens to append before attending (sdv_paged_attention_append).
struct AppendIn {
  const void* k_new;
  const void* v_new;
  const int32_t* slot_mapping;
  int64_t layer_stride;
  int32_t scale_mode;
};

static int attention(const void* q, const void* k_pages, const void* v_pages, const float* v_scales,
                     int32_t num_blocks, int64_t k_layer_stride, int64_t v_layer_stride, int64_t s_layer_stride,
                     const int32_t* block_table, int32_t max_blocks_per_seq, const int32_t* seq_lens,
                     int32_t num_layers, int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t q_len,
                     int32_t head_dim, int32_t max_seq_len, int32_t q_token_major, void* workspace,
                     size_t workspace_bytes, void* out, void* stream, int32_t phase_mask, const AppendIn* app,
                     bool path_sized_ws = false) {
  if (phase_mask <= 0 || phase_mask > SDV_PHASE_ALL) return SDV_ERR_SHAPE;
  if (!q || !k_pages || !v_pages || !v_scales || !block_table || !out) return SDV_ERR_NULL;
  if (head_dim != 64 && head_dim != 128) return SDV_ERR_UNSUPPORTED;
  if (num_blocks <= 0 || max_blocks_per_seq <= 0) return SDV_ERR_SHAPE;
  if (q_token_major != 0 && q_token_major != 1) return SDV_ERR_SHAPE;
  Plan p;
  if (!make_plan(num_layers, batch, q_heads, kv_heads, q_len, head_dim, max_seq_len, &p)) return SDV_ERR_SHAPE;
  if (p.group && phase_mask != SDV_PHASE_ALL) return SDV_ERR_UNSUPPORTED;  // one launch: no split
  if ((int64_t)max_blocks_per_seq * kBlock < max_seq_len) return SDV_ERR_SHAPE;
  const int64_t k_page = (int64_t)num_blocks * kv_heads * kBlock * head_dim;
  const int64_t s_page = (int64_t)num_blocks * kv_heads * kBlock;
  if (num_layers > 1 && (k_layer_stride < k_page || v_layer_stride < k_page || s_layer_stride < s_page))
    return SDV_ERR_SHAPE;
  if (!workspace || !aligned(workspace, 256)) return SDV_ERR_WORKSPACE;
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
  a.scores = reinterpret_cast<uint16_t*>(ws + p.off_scores);
  a.stats = reinterpret_cast<float2*>(ws + p.off_stats);
  a.partial = reinterpret_cast<float*>(ws + p.off_partial);
  a.sync = reinterpret_cast<unsigned*>(ws);
  a.f_gb = a.f_base = a.f_layers = a.f_maxblk = 0;  // chosen at launch
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
  a.pf_parts = p.pf_parts;
  a.pf_split = p.pf_split;
  a.pf_kstar = p.pf_kstar;
  a.pf_wh = p.pf_wh;
  a.vhat = reinterpret_cast<uint4*>(ws + p.off_vhat);
  a.vh_stages = p.vh_stages;
  // RN(1/sqrt(D)): 1/sqrt(128) = 0.08838834764831845, 1/sqrt(64) = 0.125 exactly
  a.inv_sqrt_d = head_dim == 128 ? 0.08838834764831845f : 0.125f;

  a.app_k = a.app_v = nullptr;
  a.app_slots = nullptr;
  a.app_ls = 0;
  a.app_scale_mode = 0;

  // path_sized_ws: the workspace only has to hold what the chosen path touches (the
  // synchronisation area for the single launch); otherwise sdv_attention_workspace_size bytes
  size_t need = p.total;
  if (path_sized_ws && phase_mask == SDV_PHASE_ALL)
    need = head_dim == 128 ? path_workspace<128>(p, a, num_layers, app != nullptr)
                           : path_workspace<64>(p, a, num_layers, app != nullptr);
  if (workspace_bytes < need) return SDV_ERR_WORKSPACE;

  hipStream_t st = static_cast<hipStream_t>(stream);
  a.tag = next_call_tag(st);
  a.spin_limit = wait_limit();
  if (app) {
    const int64_t per_layer = (int64_t)batch * q_len * kv_heads * head_dim;
    if (!app->k_new || !app->v_new) return SDV_ERR_NULL;
    if (app->scale_mode != SDV_SCALE_DIV && app->scale_mode != SDV_SCALE_RCP) return SDV_ERR_UNSUPPORTED;
    if (num_layers > 1 && app->layer_stride < per_layer) return SDV_ERR_SHAPE;
    if (!aligned(app->k_new, 16) || !aligned(app->v_new, 16) || !aligned(app->slot_mapping, 4) ||
        (num_layers > 1 && app->layer_stride % 8 != 0))
      return SDV_ERR_ALIGN;
    // offered to the single launch, which writes the new tokens itself; launch_all declines
    // (launching nothing) when another path serves the call
    a.app_k = static_cast<const uint16_t*>(app->k_new);
    a.app_v = static_cast<const uint16_t*>(app->v_new);
    a.app_slots = app->slot_mapping;
    a.app_ls = num_layers > 1 ? app->layer_stride : 0;
    a.app_scale_mode = app->scale_mode;
  }
  const int zdim = num_layers * batch;
  auto launch = [&]() {
    return head_dim == 128 ? launch_all<128>(a, p, zdim, st, phase_mask) : launch_all<64>(a, p, zdim, st, phase_mask);
  };
  if (!launch()) {
    // other paths: the append kernel first, on the same stream, then the call without the append
    if (app->slot_mapping) {
      const int st_app = sdv_quant_append(app->v_new, app->k_new, app->slot_mapping, batch * q_len, kv_heads,
                                          head_dim, head_dim, num_layers, app->layer_stride,
                                          const_cast<void*>(k_pages), const_cast<void*>(v_pages),
                                          const_cast<float*>(v_scales), num_blocks, k_layer_stride,
                                          v_layer_stride, s_layer_stride, app->scale_mode, stream);
      if (st_app != SDV_OK) return st_app;
    } else {  // the same, with the slots taken from the block table
      const SlotTable table{block_table, max_blocks_per_seq, seq_lens, q_len, max_seq_len};
      const int st_app = quant_append_table(app->v_new, app->k_new, table, batch * q_len, kv_heads, head_dim,
                                            num_layers, app->layer_stride, const_cast<void*>(k_pages),
                                            const_cast<void*>(v_pages), const_cast<float*>(v_scales), num_blocks,
                                            k_layer_stride, v_layer_stride, s_layer_stride, app->scale_mode, stream);
      if (st_app != SDV_OK) return st_app;
    }
    a.app_k = a.app_v = nullptr;
    a.app_slots = nullptr;
    if (!launch()) return SDV_ERR_HIP;  // unreachable: without a.app_v every path launches
  }
  return hipGetLastError() == hipSuccess ? SDV_OK : SDV_ERR_HIP;
}

extern "C" int sdv_paged_attention_phases(const void* q, const void* k_pages, const void* v_pages,
                                          const float* v_scales, int32_t num_blocks, int64_t k_layer_stride,
                                          int64_t v_layer_stride, int64_t s_layer_stride,
                                          const int32_t* block_table, int32_t max_blocks_per_seq,
                                          const int32_t* seq_lens, int32_t num_layers, int32_t batch,
                                          int32_t q_heads, int32_t kv_heads, int32_t q_len, int32_t head_dim,
                                          int32_t max_seq_len, int32_t q_token_major, void* workspace,
                                          size_t workspace_bytes, void* out, void* stream, int32_t phase_mask) {
  return attention(q, k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride, s_layer_stride,
                   block_table, max_blocks_per_seq, seq_lens, num_layers, batch, q_heads, kv_heads, q_len,
                   head_dim, max_seq_len, q_token_major, workspace, workspace_bytes, out, stream, phase_mask,
                   nullptr);
}

extern "C" int sdv_paged_attention_append(const void* q, const void* k_pages, const void* v_pages,
                                          const float* v_scales, int32_t num_blocks, int64_t k_layer_stride,
                                          int64_t v_layer_stride, int64_t s_layer_stride,
                                          const int32_t* block_table, int32_t max_blocks_per_seq,
                                          const int32_t* seq_lens, int32_t num_layers, int32_t batch,
                                          int32_t q_heads, int32_t kv_heads, int32_t q_len, int32_t head_dim,
                                          int32_t max_seq_len, int32_t q_token_major, void* workspace,
                                          size_t workspace_bytes, void* out, const void* k_new, const void* v_new,
                                          const int32_t* slot_mapping, int64_t new_layer_stride,
                                          int32_t scale_mode, void* stream) {
  const AppendIn app{k_new, v_new, slot_mapping, new_layer_stride, scale_mode};
  return attention(q, k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride, s_layer_stride,
                   block_table, max_blocks_per_seq, seq_lens, num_layers, batch, q_heads, kv_heads, q_len,
                   head_dim, max_seq_len, q_token_major, workspace, workspace_bytes, out, stream, SDV_PHASE_ALL,
                   &app);
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


// ---------------------------------------------------------------------------- no-allocation entry point
// Device-resident workspace for sdv_paged_attention_noalloc: one copy per GPU the library runs
// on, held until the process ends.  Host code never passes `scratch` itself to a kernel (in
// host code the name is only a stand-in for the symbol): each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kScratchBytes = (size_t)SDV_NOALLOC_MAX_WORKSPACE;
static_assert(kScratchBytes >= kSyncBytes && kScratchBytes % 256 == 0, "scratch holds the synchronisation area");
__device__ __align__(256) unsigned char scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// This device's scratch address; the first call on a device takes the symbol's address and
// zeroes its synchronisation area (a fill kernel on `st`, then waits for it), which cannot be
// recorded into a graph.
static int scratch_for_device(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return SDV_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
      (void)hipGetLastError();
      return SDV_ERR_HIP;
    }
    if (cs != hipStreamCaptureStatusNone) return SDV_ERR_UNSUPPORTED;
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      return SDV_ERR_HIP;
    }
    hipLaunchKernelGGL(zero_kernel, dim3(256), dim3(256), 0, st, static_cast<uint32_t*>(ptr), kSyncBytes / 4);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
      (void)hipGetLastError();
      return SDV_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SDV_OK;
}

extern "C" int sdv_paged_attention_noalloc(const void* q, const void* k_pages, const void* v_pages,
                                           const float* v_scales, int32_t num_blocks, int64_t k_layer_stride,
                                           int64_t v_layer_stride, int64_t s_layer_stride,
                                           const int32_t* block_table, int32_t max_blocks_per_seq,
                                           const int32_t* seq_lens, int32_t num_layers, int32_t batch,
                                           int32_t q_heads, int32_t kv_heads, int32_t q_len, int32_t head_dim,
                                           int32_t max_seq_len, int32_t q_token_major, void* out, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = scratch_for_device(st, &ws);
  if (rc != SDV_OK) return rc;
  return attention(q, k_pages, v_pages, v_scales, num_blocks, k_layer_stride, v_layer_stride, s_layer_stride,
                   block_table, max_blocks_per_seq, seq_lens, num_layers, batch, q_heads, kv_heads, q_len, head_dim,
                   max_seq_len, q_token_major, ws, kScratchBytes, out, stream, SDV_PHASE_ALL, nullptr,
                   /*path_sized_ws=*/true);
}

// A NULL workspace in sdv_attention_workspace_init / _status names the current device's
// no-allocation scratch (the workspace of sdv_paged_attention_noalloc), so its failure count
// and graph poison can be read and cleared like a caller's workspace.
static int resolve_workspace(void*& workspace, size_t& workspace_bytes, hipStream_t st) {
  if (workspace) return SDV_OK;
  const int rc = scratch_for_device(st, &workspace);
  workspace_bytes = kScratchBytes;
  return rc;
}

extern "C" int sdv_attention_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rc = resolve_workspace(workspace, workspace_bytes, st);
  if (rc != SDV_OK) return rc;
  if (!aligned(workspace, 256) || workspace_bytes < kSyncBytes) return SDV_ERR_WORKSPACE;
  hipLaunchKernelGGL(zero_kernel, dim3(256), dim3(256), 0, st, static_cast<uint32_t*>(workspace), kSyncBytes / 4);
  return hipGetLastError() == hipSuccess ? SDV_OK : SDV_ERR_HIP;
}

extern "C" int sdv_attention_workspace_status(const void* workspace, size_t workspace_bytes, uint32_t* failures,
                                              uint32_t* poisoned, void* stream) {
  if (!failures || !poisoned) return SDV_ERR_NULL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = const_cast<void*>(workspace);
  const int rc = resolve_workspace(ws, workspace_bytes, st);
  if (rc != SDV_OK) return rc;
  if (!aligned(ws, 256) || workspace_bytes < kSyncBytes) return SDV_ERR_WORKSPACE;
  uint32_t head[2] = {0, 0};
  if (hipMemcpyAsync(head, ws, sizeof(head), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    return SDV_ERR_HIP;
  }
  *failures = head[0];
  *poisoned = head[1];
  return SDV_OK;
}

extern "C" int sdv_attention_set_wait_limit(uint32_t polls) {
  g_wait_limit.store(polls, std::memory_order_relaxed);
  return SDV_OK;
}

#ifdef SDV_PHASE_TRACE
// Trace builds only: copies the phase stamps of the last single launch (workgroup i's stamps at
// words [16 i, 16 i + 10)) to host memory; synchronous on the current device.
extern "C" int sdv_phase_trace_read(unsigned long long* dst, size_t words) {
  if (!dst) return SDV_ERR_NULL;
  if (words > (size_t)kPhaseTraceGroups * kPhaseSlots) return SDV_ERR_SHAPE;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(phase_trace), words * 8, 0, hipMemcpyDeviceToHost) == hipSuccess
             ? SDV_OK
             : SDV_ERR_HIP;
}
#endif

extern "C" int32_t sdv_attention_single_launch(int32_t num_layers, int32_t batch, int32_t q_heads, int32_t kv_heads,
                                              int32_t q_len, int32_t head_dim, int32_t max_seq_len) {
  if (head_dim != 64 && head_dim != 128) return 0;
  Plan p;
  if (!make_plan(num_layers, batch, q_heads, kv_heads, q_len, head_dim, max_seq_len, &p)) return 0;
  const int R = (q_heads / kv_heads) * q_len;
  const int psl = (batch > 1 && batch <= kWave) ? num_layers : 0;  // a batch is taken to pass its lengths
  return head_dim == 128 ? fused_grid_for<128>(p, R, max_seq_len, psl) : fused_grid_for<64>(p, R, max_seq_len, psl);
}

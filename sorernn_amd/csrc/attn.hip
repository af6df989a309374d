// Gated global attention layer of the hybrid block pair for gfx950: the q/k RMSNorm + partial RoPE
// prologue and a causal GQA flash-attention forward with the sigmoid output gate fused into its
// store. Counterpart of GatedAttention.forward (sore/model/attention.py:98-135) between its
// projections: q_norm / k_norm (layers.py:7-18), PartialRotary (rope.py:24-41), then
// F.scaled_dot_product_attention(is_causal, enable_gqa) or the document-causal mask with
// cu_seqlens (attention.py:124-135), then o * sigmoid(gate) (attention.py:122).
//
// gated_attn_flash_fwd_kernel: one workgroup of 4 waves per (128-query tile, q head, batch row);
// wave w owns queries 32w..32w+31 of the tile. Per 64-key block (K and V loaded from HBM straight
// into LDS by buffer_load ... lds, double buffered, the next block's loads in flight during the
// current block's math; rows unpadded with an XOR swizzle of their 16-byte chunks):
//   S^T = K Q^T   v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = the wave's Q rows held in
//                 registers for the whole loop. The transposed product puts one query in each
//                 lane's accumulator column (lane (h, i): query i, keys 8j + 4h + r of a 32-key
//                 tile), so the online-softmax row max is an in-lane max plus one lane^32 exchange
//                 and the rescale of O^T is a per-lane scalar.
//   O^T += V^T P^T  A = V^T through ds_read_b64_tr_b16 (4 consecutive keys of one d column per
//                 read), B = P^T straight from the S^T accumulators rounded to bf16: the contraction
//                 over the block's keys runs in the order {16s + 4h + r, 16s + 8 + 4h + r}, which is
//                 the accumulator's own key order, so P never passes through LDS.
// The softmax runs on raw scores: p = 2^(s c - m c), c = scale log2(e), one FMA and one v_exp_f32 per
// score. The reference max m of a row starts at -inf (a row whose keys are all masked so far uses 0,
// no inf - inf) and moves only when a block's max exceeds it by more than 8 / c, so O^T and the row
// sum are rescaled in the first blocks and rarely after; the row sum adds the bf16-rounded p that the
// PV product uses.
// Tiles are dispatched longest first over all heads (the last query tiles have the most keys under
// the causal mask), the q heads of one kv head on one XCD; with cu_seqlens a tile may straddle
// documents and every query masks keys before its own document's start.

#include <type_traits>

#include "gdn_mfma.h"

namespace gdn {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Start of the document holding token t (t in [0, T)): the largest cu[n] <= t.
__device__ __forceinline__ int64_t doc_start_of(const void* cu, int cu_i32, int64_t n_docs, int64_t t) {
  int64_t lo = 0, hi = n_docs - 1;  // invariant: cu[lo] <= t
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (load_index(cu, cu_i32, mid) <= t) lo = mid;
    else hi = mid - 1;
  }
  return load_index(cu, cu_i32, lo);
}

// ------------------------------------------------------------------------------------------------
// q/k RMSNorm + partial rotary embedding (GPT-NeoX rotate_half on the first `rot` dims).
// One workgroup per 4 tokens: their rot/2 cos/sin pairs are computed once into LDS, then every q and
// k head row of the tokens is normalised and rotated, D/8 lanes per row (one 16-byte chunk each),
// the loads of 4 passes over the rows issued before their math.
// The reference's rounding points are kept: RMSNorm in fp32 rounded to the activation dtype
// (layers.py:15-17), cos/sin computed in fp32 and rounded to the activation dtype (rope.py:29-34),
// then x*cos and rotate_half(x)*sin each rounded before their sum is rounded (rope.py:36-40, bf16
// tensor arithmetic).
struct RopeParams {
  const bf16 *q_in, *k_in;
  int64_t q_stride, k_stride;  // elements between consecutive tokens of q_in / k_in
  const void *qw, *kw;         // RMSNorm weights [D]
  int w_dtype;
  bf16 *q_out, *k_out;         // [B, T, H, D] contiguous
  const void* cu;
  int cu_i32;
  int64_t B, T, HQ, HKV, N;
  int rot;
  float theta, eps;
};

constexpr int kRopeTokens = 4;  // tokens per workgroup

template <int D>
__global__ __launch_bounds__(256) void gated_attn_qk_norm_rope_elementwise_kernel(RopeParams p) {
  constexpr int LPR = D / 8;        // lanes per row
  constexpr int RPP = 256 / LPR;    // rows per pass of the workgroup
  constexpr int NP = 4;             // passes whose loads are issued together
  __shared__ float cs[kRopeTokens][2][D / 2];  // bf16-rounded cos / sin of each frequency, per token
  const int64_t bt0 = (int64_t)blockIdx.x * kRopeTokens;  // first flat token (batch row * T + t)
  const int64_t ntok = p.B * p.T;
  const int half = p.rot >> 1;
  const int li = threadIdx.x % LPR, d0 = 8 * li, lane = threadIdx.x % kWave;
  const int64_t hs = p.HQ + p.HKV, rows = kRopeTokens * hs;  // rows of the workgroup: token-major
  const bool lo = d0 < half, in_rot = d0 < p.rot;
  const int src_lane = in_rot ? (lo ? lane + (half >> 3) : lane - (half >> 3)) : lane;
  // the loads of a group of NP passes over the rows (rows past the end re-read a valid row)
  auto load_rows = [&](int64_t r0, bf16x8 (&xv)[NP]) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      int64_t r = r0 + u * RPP;
      r = r < rows ? r : rows - 1;
      int64_t bt = bt0 + r / hs;
      bt = bt < ntok ? bt : ntok - 1;
      const int64_t hh = r % hs;
      const bf16* src = hh < p.HQ ? p.q_in + bt * p.q_stride + hh * D : p.k_in + bt * p.k_stride + (hh - p.HQ) * D;
      xv[u] = *reinterpret_cast<const bf16x8*>(src + d0);
    }
  };
  bf16x8 xv[NP];
  int64_t r0 = threadIdx.x / LPR;
  load_rows(r0, xv);  // in flight while the cos/sin table is computed
  float wq[8], wk[8];  // this lane's 8 RMSNorm weights of q and of k
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wq[e] = load_as_f32(p.qw, p.w_dtype, d0 + e);
    wk[e] = load_as_f32(p.kw, p.w_dtype, d0 + e);
  }
  if ((int)threadIdx.x < kRopeTokens * half) {
    const int tk = threadIdx.x / half, f = threadIdx.x % half;
    const int64_t bt = bt0 + tk < ntok ? bt0 + tk : ntok - 1;
    int64_t pos = bt % p.T;
    if (p.cu) pos = bt - doc_start_of(p.cu, p.cu_i32, p.N, bt);
    const float inv = 1.f / powf(p.theta, (float)(2 * f) / (float)p.rot);
    float sv, cv;
    sincosf((float)pos * inv, &sv, &cv);
    cs[tk][0][f] = (float)(bf16)cv;
    cs[tk][1][f] = (float)(bf16)sv;
  }
  __syncthreads();
  for (; r0 < rows; r0 += NP * RPP) {  // uniform inside a row's lane group
    if (r0 != threadIdx.x / LPR) load_rows(r0, xv);
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int64_t r = r0 + u * RPP;
      if (r >= rows) break;  // uniform inside the row's lane group
      const int tk = (int)(r / hs);
      const int64_t bt = bt0 + tk, hh = r % hs;
      const bool is_q = hh < p.HQ;
      float x[8], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = (float)xv[u][e];
        ss += x[e] * x[e];
      }
      ss = group_sum<LPR>(ss);
      const float rr = __builtin_amdgcn_rsqf(ss / (float)D + p.eps);  // torch.rsqrt in the reference
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (float)(bf16)(x[e] * rr * (is_q ? wq[e] : wk[e]));
      // rotate_half partner: element d < half pairs with d + half, i.e. lane li with li +- half/8
      float py[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) py[e] = __shfl(y[e], src_lane, kWave);
      bf16x8 ov;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float o = y[e];
        if (in_rot) {
          const int f = (lo ? d0 : d0 - half) + e;
          const float rv = lo ? -py[e] : py[e];  // rotate_half(x) = cat(-x[half:rot], x[:half])
          o = (float)(bf16)((float)(bf16)(y[e] * cs[tk][0][f]) + (float)(bf16)(rv * cs[tk][1][f]));
        }
        ov[e] = (bf16)o;
      }
      if (bt < ntok) {
        bf16* dst = is_q ? p.q_out + (bt * p.HQ + hh) * D : p.k_out + (bt * p.HKV + (hh - p.HQ)) * D;
        *reinterpret_cast<bf16x8*>(dst + d0) = ov;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
struct AttnParams {
  const bf16 *q, *k, *v, *gate;
  bf16* o;
  const void* cu;
  int cu_i32;
  int64_t B, T, HQ, HKV, N;
  int64_t v_stride, gate_stride;  // elements between consecutive tokens of v / gate
  float scale_log2;               // softmax scale * log2(e)
};

constexpr int kAttnBM = 128;  // queries per workgroup
constexpr int kAttnBN = 64;   // keys per block
constexpr int kAttnNT = 256;

template <int D>
__global__ __launch_bounds__(kAttnNT, 2) void gated_attn_flash_fwd_kernel(AttnParams p) {
  constexpr int DS = D / 16;  // k-steps of S^T over the head dim
  constexpr int DT = D / 32;  // 32-row d tiles of O^T
  constexpr int LPT = kAttnBN * D / 8 / kAttnNT;  // 1 KB LDS-DMA loads per wave per K (or V) block
  constexpr int RPL = 512 / D;                   // K/V rows per 1 KB load
  __shared__ __align__(16) bf16 Ks0[kAttnBN * D];
  __shared__ __align__(16) bf16 Ks1[kAttnBN * D];
  __shared__ __align__(16) bf16 Vs0[kAttnBN * D];
  __shared__ __align__(16) bf16 Vs1[kAttnBN * D];
  // K/V rows sit unpadded in LDS (the DMA writes 1 KB contiguously per wave instruction); the 16-byte
  // chunk c of row r is stored at chunk c ^ swz(r), which keeps the K row-fragment reads and the V
  // transposed reads free of bank conflicts
  auto swz = [](int r) { return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : (((r & 3) << 1) | ((r >> 2) & 1)); };

  // w is read back as a scalar, so everything derived from it (the wave's query range, its masks
  // and skips) is wave-uniform and its branches are scalar
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), hh = lane >> 5, li = lane & 31;
  // Flat grid, longest query tiles first across all heads: workgroup rank = tile rank (slow) x
  // (q head, batch row) (fast). Workgroup i runs on XCD i % 8; when the (kv head, batch row) groups
  // divide evenly over the 8 XCDs, the q heads of one group (which read the same K/V) share an XCD
  // and its L2.
  const int64_t n_tiles = (p.T + kAttnBM - 1) / kAttnBM;
  const int rep = (int)(p.HQ / p.HKV);
  const int64_t groups = p.HKV * p.B, idx = blockIdx.x;
  int64_t rank, grp;
  int hm;
  if (groups % 8 == 0) {
    const int64_t x = idx % 8, j = idx / 8, per_xcd = (groups / 8) * rep;
    rank = j / per_xcd;
    const int64_t m = j % per_xcd;
    grp = x + 8 * (m / rep);
    hm = (int)(m % rep);
  } else {
    rank = idx / (groups * rep);
    const int64_t m = idx % (groups * rep);
    grp = m / rep;
    hm = (int)(m % rep);
  }
  const int64_t tile = n_tiles - 1 - rank;
  const int64_t b = grp / p.HKV;
  const int hkv = (int)(grp % p.HKV), hq = hkv * rep + hm;
  const int64_t q0 = tile * kAttnBM;
  const int64_t q_last = (q0 + kAttnBM < p.T ? q0 + kAttnBM : p.T) - 1;

  // this lane's query and the start of its document
  const int64_t qi = q0 + 32 * w + li;
  const bool q_ok = qi < p.T;
  const int64_t qi_c = q_ok ? qi : p.T - 1;
  const int64_t ds_q = p.cu ? doc_start_of(p.cu, p.cu_i32, p.N, qi_c) : 0;
  // the wave's query range and the smallest / largest document start in it (monotone in the query)
  const int64_t wq0 = q0 + 32 * w, wq1 = (wq0 + 31 < q_last ? wq0 + 31 : q_last);
  const bool wave_live = wq0 <= q_last;
  const int64_t wds0 = p.cu && wave_live ? doc_start_of(p.cu, p.cu_i32, p.N, wq0) : 0;
  const int64_t wds1 = p.cu && wave_live ? doc_start_of(p.cu, p.cu_i32, p.N, wq1) : 0;
  const int64_t kv_lo = p.cu ? doc_start_of(p.cu, p.cu_i32, p.N, q0) : 0;
  const int64_t jb0 = kv_lo / kAttnBN, jb1 = q_last / kAttnBN + 1;

  // Q^T fragments (B operand of S^T): lane (hh, li) holds query qi, d = 16s + 8hh .. +7
  const int64_t rowq = p.HQ * D, rowk = p.HKV * D;
  bf16x8 qf[DS];
  {
    const auto rq = make_rsrc(p.q + (b * p.T * p.HQ + hq) * D, (uint32_t)(p.T * rowq * 2));
#pragma unroll
    for (int s = 0; s < DS; ++s) qf[s] = buf_load16(rq, (uint32_t)((qi * rowq + 16 * s + 8 * hh) * 2));
    if (!q_ok) {
#pragma unroll
      for (int s = 0; s < DS; ++s) qf[s] = bf16x8{};
    }
  }

  // K/V blocks go from HBM straight into LDS (buffer_load ... lds): load u of wave w fills LDS bytes
  // [(w + 4u) KB, +1 KB) of the block, lane l the 16 bytes at l * 16, i.e. row (w + 4u) RPL + l / (D/8),
  // chunk slot l % (D/8), which receives the source chunk slot ^ swz(row). The swizzle of a lane's
  // row does not depend on w or u, so the per-lane source offset is a loop constant plus a scalar step.
  // Each block gets buffer resources based at its first key and sized to the keys left in the
  // sequence; keys past the end are masked for every query.
  const bf16* const kbase = p.k + (b * p.T * p.HKV + hkv) * D;
  const bf16* const vbase = p.v + b * p.T * p.v_stride + (int64_t)hkv * D;
  const int drow = w * RPL + lane / (D / 8), dslot = lane % (D / 8), dch = dslot ^ swz(drow);
  const uint32_t koff = (uint32_t)((drow * rowk + dch * 8) * 2), voff = (uint32_t)((drow * p.v_stride + dch * 8) * 2);
  const uint32_t kstep = (uint32_t)(4 * RPL * rowk * 2), vstep = (uint32_t)(4 * RPL * p.v_stride * 2);
  auto fetch = [&](int64_t jb, bf16* kd, bf16* vd) {
    const int64_t key0 = jb * kAttnBN, left = p.T - key0 > 0 ? p.T - key0 : 0;
    const auto rk = make_rsrc(kbase + key0 * rowk, (uint32_t)(left * rowk * 2));
    const auto rv = make_rsrc(vbase + key0 * p.v_stride, (uint32_t)(left * p.v_stride * 2));
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(kd + (w + 4 * u) * 512), 16,
                                               koff + u * kstep, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(vd + (w + 4 * u) * 512), 16,
                                               voff + u * vstep, 0, 0, 0);
    }
  };
  // the wave's own LDS-DMA loads have landed (vmcnt(0)); the barrier after it publishes them
  auto dma_wait = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };
  // K row-fragment and V transposed-read offsets (elements) inside a block buffer: K row 32kt + li,
  // chunk 2st + hh; V rows 16ks + 4hh + lm (+ 8), chunk 4d + 2gsub + lq / 2, half lq % 2
  const int gsub = (lane >> 4) & 1, lm = (lane & 15) >> 2, lq = lane & 3;
  int kq_off[DS], v_off[DT][2];
#pragma unroll
  for (int st = 0; st < DS; ++st) kq_off[st] = li * D + (((2 * st + hh) ^ swz(li)) << 3);
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int h8 = 0; h8 < 2; ++h8) {
      const int row = 4 * hh + lm + 8 * h8;
      v_off[d][h8] = row * D + (((4 * d + 2 * gsub + (lq >> 1)) ^ swz(row)) << 3) + 4 * (lq & 1);
    }
  if (p.T % kAttnBN) {  // a partial last block: rows past the end read as zeros from a cleared buffer
    for (int e = t; e < kAttnBN * D / 8; e += kAttnNT) {
      reinterpret_cast<bf16x8*>(Ks0)[e] = bf16x8{};
      reinterpret_cast<bf16x8*>(Ks1)[e] = bf16x8{};
      reinterpret_cast<bf16x8*>(Vs0)[e] = bf16x8{};
      reinterpret_cast<bf16x8*>(Vs1)[e] = bf16x8{};
    }
    __syncthreads();
  }

  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  const float lazy_thr = 8.f / p.scale_log2;

  // One 64-key block of the wave's 32 queries. `masked` (wave-uniform, a scalar branch) applies the
  // causal / document mask; blocks strictly below every query of the wave and inside every query's
  // document skip it.
  auto block = [&](bool masked, const bf16* kb, const bf16* vb, int64_t k0) {
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x16{};
#pragma unroll
      for (int st = 0; st < DS; ++st)
        s[kt] = mfma32(ld8(kb + 32 * kt * D + kq_off[st]), qf[st], s[kt]);
    }
    if (masked) {  // 32-bit key offsets inside the block against this lane's limits
      const int hi_lim = (int)(qi - k0), lo_lim = (int)(ds_q - k0);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int ko = 32 * kt + 8 * (e >> 2) + 4 * hh + (e & 3);
          if (ko > hi_lim || ko < lo_lim) s[kt][e] = -INFINITY;
        }
    }
    // online softmax on the raw scores (scale > 0 commutes with the max): p = 2^(s c - m c) with
    // c = scale log2(e), one FMA and one v_exp_f32 per score. The reference max m of a row moves only
    // when a block max exceeds it by more than 8 / c (p <= 2^8 meanwhile), so O^T is rescaled in the
    // first blocks and then rarely; a row whose keys are all masked so far keeps m = -inf and uses 0.
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float c = p.scale_log2;
    const bool grow = mx > m_run + lazy_thr;
    if (!__all(!grow)) {
      const float alpha = grow ? __builtin_amdgcn_exp2f((m_run - mx) * c) : 1.f;  // 0 while no key was seen
      m_run = grow ? mx : m_run;
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DT; ++d) acc[d] *= alpha;
    }
    const float nmc = m_run == -INFINITY ? 0.f : -m_run * c;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kt][e] = __builtin_amdgcn_exp2f(fmaf(s[kt][e], c, nmc));
    // P^T as B operands: k-step ks covers keys 16ks + {4hh + r, 8 + 4hh + r}; the row sum adds the
    // bf16-rounded p (the values the PV product uses), two per v_dot2_f32_bf16
    bf16x8 pb[4];
    float rs = 0.f;
    const bf16x2 ones = {(bf16)1.f, (bf16)1.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kt = ks >> 1, j0 = 2 * (ks & 1);
      pb[ks] = bf16x8{(bf16)s[kt][4 * j0], (bf16)s[kt][4 * j0 + 1], (bf16)s[kt][4 * j0 + 2], (bf16)s[kt][4 * j0 + 3],
                      (bf16)s[kt][4 * j0 + 4], (bf16)s[kt][4 * j0 + 5], (bf16)s[kt][4 * j0 + 6], (bf16)s[kt][4 * j0 + 7]};
#pragma unroll
      for (int h2 = 0; h2 < 4; ++h2) rs = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{pb[ks][2 * h2], pb[ks][2 * h2 + 1]}, ones, rs, false);
    }
    l_run += rs;
    // V^T A operands: lane 4m + q of 16-lane group G reads row 16ks + 4hh + m (then + 8) at
    // columns 32d + 16(G & 1) + 4q, and receives V[16ks + 4hh + m'][32d + li], m' = 0..3
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const bf16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vb + 16 * ks * D + v_off[d][0]));
        const bf16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vb + 16 * ks * D + v_off[d][1]));
        acc[d] = mfma32(bf16x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]}, pb[ks], acc[d]);
      }
  };

  // one key block on the buffers (kc, vc) while the next block is loaded into (kn, vn); the two
  // buffer pairs alternate through a loop unrolled by two, so every LDS access names its array
  auto step = [&](int64_t jb, const bf16* kc, const bf16* vc, bf16* kn, bf16* vn) {
    if (jb + 1 < jb1) fetch(jb + 1, kn, vn);
    const int64_t k0 = jb * kAttnBN;
    // keys of the block beyond every query of the wave, or before every query's document: skip;
    // keys after some query or before some query's document: mask (both conditions wave-uniform)
    if (wave_live && k0 <= wq1 && k0 + kAttnBN > wds0) {
      block((k0 + kAttnBN - 1 > wq0) || (k0 < wds1), kc, vc, k0);
    }
    dma_wait();
    __syncthreads();
  };
  fetch(jb0, Ks0, Vs0);
  dma_wait();
  __syncthreads();
  for (int64_t jb = jb0; jb < jb1; jb += 2) {
    step(jb, Ks0, Vs0, Ks1, Vs1);
    if (jb + 1 < jb1) step(jb + 1, Ks1, Vs1, Ks0, Vs0);
  }

  // epilogue: O = O^T / l * sigmoid(gate); lane (hh, li) holds query qi, d = 32d + 8j + 4hh + r
  if (!q_ok) return;
  const float l = l_run + __shfl_xor(l_run, 32, kWave);
  const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
  const bf16* gp = p.gate + (b * p.T + qi) * p.gate_stride + (int64_t)hq * D;
  bf16* op = p.o + ((b * p.T + qi) * p.HQ + hq) * D;
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 32 * d + 8 * j + 4 * hh;
      const bf16x4 gv = *reinterpret_cast<const bf16x4*>(gp + c);
      float ov[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) ov[r] = acc[d][4 * j + r] * inv * __builtin_amdgcn_rcpf(1.f + __expf(-(float)gv[r]));
      *reinterpret_cast<bf16x4*>(op + c) = to_bf16x4(ov[0], ov[1], ov[2], ov[3]);
    }
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_attn_qk_norm_rope_fwd(const void* q_in, int64_t q_row_stride, const void* k_in,
                                         int64_t k_row_stride, const void* q_weight, const void* k_weight,
                                         int w_dtype, void* q_out, void* k_out, const void* cu_seqlens, int64_t B,
                                         int64_t T, int64_t HQ, int64_t HKV, int64_t D, int64_t N, int rot_dim,
                                         float theta, float eps, unsigned flags, void* stream) {
  if (!q_in || !k_in || !q_weight || !k_weight || !q_out || !k_out) {
    gdn_internal_set_error("gdn_attn_qk_norm_rope_fwd: null pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || HQ <= 0 || HKV <= 0 || N <= 0 || (cu_seqlens ? B != 1 : N != B)) {
    gdn_internal_set_error("gdn_attn_qk_norm_rope_fwd: bad sizes B=%lld T=%lld HQ=%lld HKV=%lld N=%lld "
                           "(cu_seqlens requires B == 1)", (long long)B, (long long)T, (long long)HQ,
                           (long long)HKV, (long long)N);
    return GDN_ERR_INVALID;
  }
  if ((D != 64 && D != 128) || rot_dim <= 0 || rot_dim > D || rot_dim % 16) {
    gdn_internal_set_error("gdn_attn_qk_norm_rope_fwd: D=%lld rot_dim=%d unsupported (D = 64 or 128, rot_dim a "
                           "positive multiple of 16 <= D)", (long long)D, rot_dim);
    return GDN_ERR_UNSUPPORTED;
  }
  if (q_row_stride < HQ * D || k_row_stride < HKV * D || q_row_stride % 8 || k_row_stride % 8 ||
      ((reinterpret_cast<uintptr_t>(q_in) | reinterpret_cast<uintptr_t>(k_in)) & 15)) {
    gdn_internal_set_error("gdn_attn_qk_norm_rope_fwd: row strides %lld/%lld too small or not 16-byte aligned",
                           (long long)q_row_stride, (long long)k_row_stride);
    return GDN_ERR_INVALID;
  }
  if (w_dtype != GDN_DTYPE_F32 && w_dtype != GDN_DTYPE_BF16) {
    gdn_internal_set_error("gdn_attn_qk_norm_rope_fwd: weight dtype %d unsupported (fp32 or bf16)", w_dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  if (B * T == 0) return GDN_OK;
  if (B * T > 0x7fffffffLL) {
    gdn_internal_set_error("gdn_attn_qk_norm_rope_fwd: B*T=%lld exceeds the grid", (long long)(B * T));
    return GDN_ERR_UNSUPPORTED;
  }
  RopeParams p{static_cast<const bf16*>(q_in), static_cast<const bf16*>(k_in), q_row_stride, k_row_stride,
               q_weight, k_weight, w_dtype, static_cast<bf16*>(q_out), static_cast<bf16*>(k_out), cu_seqlens,
               (flags & GDN_FLAG_CU_INT32) ? 1 : 0, B, T, HQ, HKV, N, rot_dim, theta, eps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((B * T + kRopeTokens - 1) / kRopeTokens));
  if (D == 128) hipLaunchKernelGGL(gated_attn_qk_norm_rope_elementwise_kernel<128>, grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL(gated_attn_qk_norm_rope_elementwise_kernel<64>, grid, dim3(256), 0, s, p);
  return gdn_internal_check_launch("gated_attn_qk_norm_rope_elementwise_kernel");
}

extern "C" int gdn_attn_fwd(const void* q, const void* k, const void* v, int64_t v_row_stride, const void* gate,
                            int64_t gate_row_stride, void* o, const void* cu_seqlens, int64_t B, int64_t T,
                            int64_t HQ, int64_t HKV, int64_t D, int64_t N, float scale, unsigned flags,
                            void* stream) {
  if (!q || !k || !v || !gate || !o) {
    gdn_internal_set_error("gdn_attn_fwd: null pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || HQ <= 0 || HKV <= 0 || HQ % HKV || N <= 0 || (cu_seqlens ? B != 1 : N != B)) {
    gdn_internal_set_error("gdn_attn_fwd: bad sizes B=%lld T=%lld HQ=%lld HKV=%lld N=%lld (HQ a multiple of HKV; "
                           "cu_seqlens requires B == 1)", (long long)B, (long long)T, (long long)HQ, (long long)HKV,
                           (long long)N);
    return GDN_ERR_INVALID;
  }
  if (D != 64 && D != 128) {
    gdn_internal_set_error("gdn_attn_fwd: head dim %lld unsupported (64 or 128)", (long long)D);
    return GDN_ERR_UNSUPPORTED;
  }
  if (!(scale > 0.f) || scale > 3.0e38f) {
    gdn_internal_set_error("gdn_attn_fwd: scale %g unsupported (a positive finite softmax scale)", (double)scale);
    return GDN_ERR_INVALID;
  }
  if (v_row_stride < HKV * D || gate_row_stride < HQ * D || v_row_stride % 8 || gate_row_stride % 4) {
    gdn_internal_set_error("gdn_attn_fwd: v/gate row strides %lld/%lld too small or misaligned",
                           (long long)v_row_stride, (long long)gate_row_stride);
    return GDN_ERR_INVALID;
  }
  // buffer resources address each (batch row, head) slab with 32-bit byte offsets
  if (T * (HQ > HKV ? HQ : HKV) * D * 2 > 0x7fffffffLL || T * v_row_stride * 2 > 0x7fffffffLL) {
    gdn_internal_set_error("gdn_attn_fwd: sequence too long for 32-bit offsets (T=%lld)", (long long)T);
    return GDN_ERR_UNSUPPORTED;
  }
  if (T == 0) return GDN_OK;
  AttnParams p{static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
               static_cast<const bf16*>(gate), static_cast<bf16*>(o), cu_seqlens,
               (flags & GDN_FLAG_CU_INT32) ? 1 : 0, B, T, HQ, HKV, N, v_row_stride, gate_row_stride,
               scale * 1.4426950408889634f};
  const int64_t wgs = ((T + kAttnBM - 1) / kAttnBM) * HQ * B;
  if (wgs > 0x7fffffffLL) {
    gdn_internal_set_error("gdn_attn_fwd: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)wgs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) hipLaunchKernelGGL(gated_attn_flash_fwd_kernel<128>, grid, dim3(kAttnNT), 0, s, p);
  else hipLaunchKernelGGL(gated_attn_flash_fwd_kernel<64>, grid, dim3(kAttnNT), 0, s, p);
  return gdn_internal_check_launch("gated_attn_flash_fwd_kernel");
}

// Gated global attention layer of the hybrid block pair for gfx950: the q/k RMSNorm + partial RoPE
// prologue and a causal GQA flash-attention forward with the sigmoid output gate fused into its
// store. Counterpart of GatedAttention.forward (sore/model/attention.py:98-135) between its
// projections: q_norm / k_norm (layers.py:7-18), PartialRotary (rope.py:24-41), then
// F.scaled_dot_product_attention(is_causal, enable_gqa) or the document-causal mask with
// cu_seqlens (attention.py:124-135), then o * sigmoid(gate) (attention.py:122).
//
// gated_attn_flash_fwd_kernel: one workgroup of 4 waves per (128-query tile, q head, batch row);
// wave w owns queries 32w..32w+31 of the tile. Per 64-key block (K and V staged through LDS, double
// buffered, the next block's global loads in flight during the current block's math):
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
// score; the running max starts at -inf and a row whose keys are all masked so far uses 0 as its max
// (no inf - inf); O^T is rescaled only in blocks where some row's max moved.
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
  constexpr int KP = D + 8;   // K row pitch: 16 consecutive rows of one 16-byte column hit distinct banks
  constexpr int VP = D + 32;  // V row pitch: the 4 rows of a transposed read sit 64 bytes apart in the banks
  constexpr int DS = D / 16;  // k-steps of S^T over the head dim
  constexpr int DT = D / 32;  // 32-row d tiles of O^T
  constexpr int LPT = kAttnBN * D / 8 / kAttnNT;  // 16-byte loads per thread per K (or V) block
  __shared__ __align__(16) bf16 Ks[2][kAttnBN * KP];
  __shared__ __align__(16) bf16 Vs[2][kAttnBN * VP];

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

  // cooperative K/V block loads: thread t handles 16-byte chunks t + 256u (row (t + 256u) / (D/8)).
  // The per-lane byte offsets inside a block are loop constants; each block gets buffer resources
  // based at its first key and sized to the keys left in the sequence, so keys past the end read as
  // zeros and no offset is recomputed per block.
  const bf16* const kbase = p.k + (b * p.T * p.HKV + hkv) * D;
  const bf16* const vbase = p.v + b * p.T * p.v_stride + (int64_t)hkv * D;
  // thread t's chunks u sit (2048 / D) rows apart: one per-lane offset plus a scalar step
  constexpr int RSTEP = kAttnNT / (D / 8);
  const uint32_t koff = (uint32_t)(((t / (D / 8)) * rowk + (t % (D / 8)) * 8) * 2);
  const uint32_t voff = (uint32_t)(((t / (D / 8)) * p.v_stride + (t % (D / 8)) * 8) * 2);
  const uint32_t kstep = (uint32_t)(RSTEP * rowk * 2), vstep = (uint32_t)(RSTEP * p.v_stride * 2);
  auto fetch = [&](int64_t jb, bf16x8 (&kr)[LPT], bf16x8 (&vr)[LPT]) {
    const int64_t key0 = jb * kAttnBN, left = p.T - key0 > 0 ? p.T - key0 : 0;
    const auto rk = make_rsrc(kbase + key0 * rowk, (uint32_t)(left * rowk * 2));
    const auto rv = make_rsrc(vbase + key0 * p.v_stride, (uint32_t)(left * p.v_stride * 2));
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      kr[u] = buf_load16(rk, koff + u * kstep);
      vr[u] = buf_load16(rv, voff + u * vstep);
    }
  };
  auto stage = [&](int buf, const bf16x8 (&kr)[LPT], const bf16x8 (&vr)[LPT]) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int c = t + kAttnNT * u, r = c / (D / 8), col = (c % (D / 8)) * 8;
      *reinterpret_cast<bf16x8*>(&Ks[buf][r * KP + col]) = kr[u];
      *reinterpret_cast<bf16x8*>(&Vs[buf][r * VP + col]) = vr[u];
    }
  };

  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

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
        s[kt] = mfma32(ld8(kb + (32 * kt + li) * KP + 16 * st + 8 * hh), qf[st], s[kt]);
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
    // c = scale log2(e), one FMA and one v_exp_f32 per score
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float c = p.scale_log2, nmc = -m_use * c;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * c);  // 0 while no key was seen
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(s[kt][e], c, nmc));
        s[kt][e] = pv;
        rs += pv;
      }
    l_run = l_run * alpha + rs;
    // the running max of most rows stops moving after the first blocks: rescale O^T only when
    // some lane's max moved (alpha != 1)
    if (!__all(alpha == 1.f)) {
#pragma unroll
      for (int d = 0; d < DT; ++d) acc[d] *= alpha;
    }
    // P^T as B operands: k-step ks covers keys 16ks + {4hh + r, 8 + 4hh + r}
    bf16x8 pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kt = ks >> 1, j0 = 2 * (ks & 1);
      pb[ks] = bf16x8{(bf16)s[kt][4 * j0], (bf16)s[kt][4 * j0 + 1], (bf16)s[kt][4 * j0 + 2], (bf16)s[kt][4 * j0 + 3],
                      (bf16)s[kt][4 * j0 + 4], (bf16)s[kt][4 * j0 + 5], (bf16)s[kt][4 * j0 + 6], (bf16)s[kt][4 * j0 + 7]};
    }
    // V^T A operands: lane 4m + q of 16-lane group G reads row 16ks + 4hh + m (then + 8) at
    // columns 32d + 16(G & 1) + 4q, and receives V[16ks + 4hh + m'][32d + li], m' = 0..3
    const int gsub = (lane >> 4) & 1, lm = (lane & 15) >> 2, lq = lane & 3;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const bf16* p0 = vb + (16 * ks + 4 * hh + lm) * VP + 32 * d + 16 * gsub + 4 * lq;
        const bf16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0));
        const bf16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 8 * VP));
        acc[d] = mfma32(bf16x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]}, pb[ks], acc[d]);
      }
  };

  {
    bf16x8 kr[LPT], vr[LPT];
    fetch(jb0, kr, vr);
    stage(0, kr, vr);
  }
  __syncthreads();
  for (int64_t jb = jb0; jb < jb1; ++jb) {
    const int buf = (int)((jb - jb0) & 1);
    bf16x8 kr[LPT], vr[LPT];
    const bool more = jb + 1 < jb1;
    if (more) fetch(jb + 1, kr, vr);
    const int64_t k0 = jb * kAttnBN;
    // keys of the block beyond every query of the wave, or before every query's document: skip;
    // keys after some query or before some query's document: mask (both conditions wave-uniform)
    if (wave_live && k0 <= wq1 && k0 + kAttnBN > wds0) {
      block((k0 + kAttnBN - 1 > wq0) || (k0 < wds1), Ks[buf], Vs[buf], k0);
    }
    if (more) stage(buf ^ 1, kr, vr);
    __syncthreads();
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

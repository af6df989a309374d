// Recurrent gated delta rule (token by token, state on chip) and the fused decode step.
//
// One workgroup of 256 threads owns one (sequence, value head) state S [K, V] fp32 for the whole
// sequence: it is read from HBM once, kept in registers (16 float4 per thread at K = V = 128) and
// written once. Thread t owns the 4 columns 4*(t % (V/4)) .. +3 and the rows rg + RG*i, where
// rg = t / (V/4) and RG = 256 / (V/4); the columns' dot products with k and q reduce over row groups
// with a cross-lane xor reduction inside each wave and one LDS exchange across the 4 waves.
// Per token (sore/model/gdn_ref.py:17-21):
//   a = exp(g), S_dec = a S, delta = beta (v - S_dec^T k), S' = S_dec + k delta^T,
//   o = scale S'^T q = scale (a S^T q + delta (k . q)),
// so one pass over S yields S^T k and S^T q together (the state is read once per token).
// No MFMA: per token the work is two matrix-vector products and a rank-1 update, bandwidth-bound.

#include "gdn_common.h"
#include "gdn_mfma.h"

namespace gdn {

struct RecParams {
  const void *q, *k, *v, *g, *beta;
  const float* h0;
  void* o;
  float* ht;
  const void* cu;
  int cu_i32;
  int64_t T, H, HV;
  int dq, dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
};

template <int KD, int VD>
struct RecLayout {
  static constexpr int NT = 256;
  static constexpr int CG = VD / 4;  // column groups of 4 columns
  static constexpr int RG = NT / CG;  // row groups
  static constexpr int RPT = KD / RG;  // rows per thread
  static constexpr int NW = NT / kWave;
  static constexpr int NRED = 11;  // S^T k (4), S^T q (4), k.q, k.k, q.q
  static_assert(CG <= kWave && RG * RPT == KD, "unsupported head dims");
};

// The thread's slice of the state: RPT rows x 4 columns, in registers.
template <int KD, int VD>
struct StateRegs {
  float4 r[RecLayout<KD, VD>::RPT];
};

// Decay and write strength of one (token, value head).
__device__ __forceinline__ void gate_values(const RecParams& p, int64_t idx, int hv, float& a, float& b) {
  float gv = load_as_f32(p.g, p.dg, idx);
  if (p.flags & GDN_FLAG_GATE_IN_KERNEL) gv = -expf(p.A_log[hv]) * softplus_f32(gv + p.dt_bias[hv]);
  a = expf(gv);
  float bv = load_as_f32(p.beta, p.db, idx);
  b = (p.flags & GDN_FLAG_BETA_SIGMOID) ? sigmoid_f32(bv) : bv;
}

// One token on the register-resident state. q_l/k_l/v_l are the token's vectors in LDS (fp32),
// red is an LDS exchange buffer of NW*CG*12 floats. Writes the 4 output columns into o4.
template <int KD, int VD>
__device__ __forceinline__ void rec_token(StateRegs<KD, VD>& sr, const float* q_l, const float* k_l,
                                          const float* v_l, float a, float b, bool l2, float scale, float* red,
                                          float (&o4)[4]) {
  using L = RecLayout<KD, VD>;
  auto& s = sr.r;
  const int t = threadIdx.x, cg = t % L::CG, rg = t / L::CG, lane = t % kWave, w = t / kWave;
  float p[L::NRED];
#pragma unroll
  for (int j = 0; j < L::NRED; ++j) p[j] = 0.f;
#pragma unroll
  for (int i = 0; i < L::RPT; ++i) {
    const int r = rg + L::RG * i;
    const float kr = k_l[r], qr = q_l[r];
    p[0] += s[i].x * kr; p[1] += s[i].y * kr; p[2] += s[i].z * kr; p[3] += s[i].w * kr;
    p[4] += s[i].x * qr; p[5] += s[i].y * qr; p[6] += s[i].z * qr; p[7] += s[i].w * qr;
    p[8] += kr * qr; p[9] += kr * kr; p[10] += qr * qr;
  }
#pragma unroll
  for (int j = 0; j < L::NRED; ++j) p[j] = wave_xor_sum(p[j], L::CG);
  if (lane < L::CG) {
#pragma unroll
    for (int j = 0; j < L::NRED; ++j) red[(w * L::CG + cg) * 12 + j] = p[j];
  }
  __syncthreads();
  float tot[L::NRED];
#pragma unroll
  for (int j = 0; j < L::NRED; ++j) {
    float x = 0.f;
#pragma unroll
    for (int ww = 0; ww < L::NW; ++ww) x += red[(ww * L::CG + cg) * 12 + j];
    tot[j] = x;
  }
  // F.normalize semantics: x / max(||x||, 1e-12)
  const float ik = l2 ? 1.f / fmaxf(sqrtf(tot[9]), 1e-12f) : 1.f;
  const float iq = l2 ? 1.f / fmaxf(sqrtf(tot[10]), 1e-12f) : 1.f;
  float d[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    d[c] = b * (v_l[4 * cg + c] - a * tot[c] * ik);
    o4[c] = scale * (a * tot[4 + c] * iq + d[c] * tot[8] * ik * iq);
  }
#pragma unroll
  for (int i = 0; i < L::RPT; ++i) {
    const float kr = k_l[rg + L::RG * i] * ik;
    s[i].x = a * s[i].x + kr * d[0];
    s[i].y = a * s[i].y + kr * d[1];
    s[i].z = a * s[i].z + kr * d[2];
    s[i].w = a * s[i].w + kr * d[3];
  }
}

template <int KD, int VD>
__device__ __forceinline__ void load_state(StateRegs<KD, VD>& sr, const float* base) {
  using L = RecLayout<KD, VD>;
  auto& s = sr.r;
  const int t = threadIdx.x, cg = t % L::CG, rg = t / L::CG;
#pragma unroll
  for (int i = 0; i < L::RPT; ++i) {
    if (base) s[i] = *reinterpret_cast<const float4*>(base + (int64_t)(rg + L::RG * i) * VD + 4 * cg);
    else s[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

template <int KD, int VD>
__device__ __forceinline__ void store_state(const StateRegs<KD, VD>& sr, float* base) {
  using L = RecLayout<KD, VD>;
  const auto& s = sr.r;
  const int t = threadIdx.x, cg = t % L::CG, rg = t / L::CG;
#pragma unroll
  for (int i = 0; i < L::RPT; ++i) *reinterpret_cast<float4*>(base + (int64_t)(rg + L::RG * i) * VD + 4 * cg) = s[i];
}

// grid (HV, N): one workgroup per (value head, sequence), tokens in order.
template <int KD, int VD>
__global__ __launch_bounds__(256) void gated_delta_recurrent_kernel(RecParams p) {
  using L = RecLayout<KD, VD>;
  __shared__ float stage[2][2 * KD + VD];
  __shared__ float red[2][L::NW * L::CG * 12];
  const int hv = blockIdx.x;
  const int64_t n = blockIdx.y;
  const int h = hv / (int)(p.HV / p.H);
  int64_t bos, eos;
  if (p.cu) {
    bos = load_index(p.cu, p.cu_i32, n);
    eos = load_index(p.cu, p.cu_i32, n + 1);
  } else {
    bos = n * p.T;
    eos = bos + p.T;
  }
  const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD;
  StateRegs<KD, VD> s;
  load_state<KD, VD>(s, p.h0 ? p.h0 + sbase : nullptr);
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const int t = threadIdx.x;
  int par = 0;
  for (int64_t tok = bos; tok < eos; ++tok, par ^= 1) {
    float* st = stage[par];
    for (int e = t; e < 2 * KD + VD; e += L::NT) {
      float x;
      if (e < KD) x = load_as_f32(p.q, p.dq, (tok * p.H + h) * KD + e);
      else if (e < 2 * KD) x = load_as_f32(p.k, p.dq, (tok * p.H + h) * KD + (e - KD));
      else x = load_as_f32(p.v, p.dq, (tok * p.HV + hv) * VD + (e - 2 * KD));
      st[e] = x;
    }
    float a, b;
    gate_values(p, tok * p.HV + hv, hv, a, b);
    __syncthreads();
    float o4[4];
    rec_token<KD, VD>(s, st, st + KD, st + 2 * KD, a, b, l2, p.scale, red[par], o4);
    if (t < L::CG) {
      const int64_t ob = (tok * p.HV + hv) * VD + 4 * t;
#pragma unroll
      for (int c = 0; c < 4; ++c) store_from_f32(p.o, p.dq, ob + c, o4[c]);
    }
  }
  if (p.ht) store_state<KD, VD>(s, p.ht + sbase);
}

struct DecodeParams {
  const void* x;
  void* conv_state;
  const float* conv_w;
  const void *g, *beta;
  float* state;
  void* o;
  int64_t H, HV, W;
  int dx, dcs, dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
};

// Conv-cache update + conv + SiLU of channel ch of batch row b; returns the activation rounded to
// the activation dtype (as a separate conv kernel would store it).
__device__ __forceinline__ float decode_conv_channel(const DecodeParams& p, int64_t b, int64_t C, int64_t ch) {
  // window = (state[1..W-1], x); y = sum_i w[ch, i] window[i]; the new state is the window.
  const int64_t cbase = (b * C + ch) * p.W;
  float acc = 0.f;
  for (int i = 1; i < p.W; ++i) {
    const float xi = load_as_f32(p.conv_state, p.dcs, cbase + i);
    acc += p.conv_w[ch * p.W + i - 1] * xi;
    store_from_f32(p.conv_state, p.dcs, cbase + i - 1, xi);  // index i-1 was read one step earlier
  }
  const float xc = load_as_f32(p.x, p.dx, b * C + ch);
  acc += p.conv_w[ch * p.W + p.W - 1] * xc;
  store_from_f32(p.conv_state, p.dcs, cbase + p.W - 1, xc);
  return round_to(p.dx, silu_f32(acc));
}

// grid (H, B): one workgroup per (q/k head, batch row). It computes the q/k conv of its head once
// (so the shared conv cache of q/k is written by exactly one workgroup) and then updates the
// HV/H value heads that read this q/k head, one after the other.
template <int D>
__global__ __launch_bounds__(256) void gated_delta_decode_kernel(DecodeParams p) {
  using L = RecLayout<D, D>;
  __shared__ float qk[2 * D];
  __shared__ float vs[2][D];
  __shared__ float red[2][L::NW * L::CG * 12];
  const int h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int rep = (int)(p.HV / p.H);
  const int64_t C = (2 * p.H + p.HV) * D;
  const int t = threadIdx.x;
  for (int e = t; e < 2 * D; e += L::NT) {
    const int64_t ch = (e < D) ? (int64_t)h * D + e : p.H * D + (int64_t)h * D + (e - D);
    qk[e] = decode_conv_channel(p, b, C, ch);
  }
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  for (int r = 0; r < rep; ++r) {
    const int hv = h * rep + r;
    const int par = r & 1;
    const int64_t sbase = (b * p.HV + hv) * (int64_t)D * D;
    StateRegs<D, D> s;
    load_state<D, D>(s, p.state + sbase);
    for (int e = t; e < D; e += L::NT) vs[par][e] = decode_conv_channel(p, b, C, 2 * p.H * D + (int64_t)hv * D + e);
    RecParams gp{};
    gp.g = p.g; gp.beta = p.beta; gp.dg = p.dg; gp.db = p.db; gp.flags = p.flags;
    gp.A_log = p.A_log; gp.dt_bias = p.dt_bias;
    float a, bb;
    gate_values(gp, b * p.HV + hv, hv, a, bb);
    __syncthreads();
    float o4[4];
    rec_token<D, D>(s, qk, qk + D, vs[par], a, bb, l2, p.scale, red[par], o4);
    if (t < L::CG) {
      const int64_t ob = (b * p.HV + hv) * D + 4 * t;
#pragma unroll
      for (int c = 0; c < 4; ++c) store_from_f32(p.o, p.dx, ob + c, o4[c]);
    }
    store_state<D, D>(s, p.state + sbase);
  }
}


template <class T>
__device__ __forceinline__ float elem_to_f32(T x) { return static_cast<float>(x); }
template <class T>
__device__ __forceinline__ T f32_to_elem(float x) { return static_cast<T>(x); }

// Width-W conv cache of one channel as one vector access (W * sizeof(T) bytes).
template <int W, class T>
struct alignas(W * sizeof(T) >= 16 ? 16 : W * sizeof(T)) ConvWindow {
  T v[W];
};

// Sum over the 8 row groups of a column group (lanes l ^ 8, l ^ 16, l ^ 32) in three VALU steps:
// DPP row_ror:8 inside each 16-lane row, then the 16- and 32-lane swaps of gfx950
__device__ __forceinline__ float rg_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Fast decode step for width-4 conv caches whose dtype equals the activation dtype T: one
// workgroup per (sequence, q/k head), looping over that head's value heads. Wave w owns the 32-column
// block w of the state (columns of the recurrence are independent: column j needs only S[:, j]), 16
// rows x 4 columns per lane, so the reductions over the state's rows (S^T k, S^T q) stay inside the
// wave and no reduction crosses waves: one barrier per value head publishes the conv outputs q, k, v
// in LDS. The four waves read their blocks at once, i.e. the whole 64 KB state, with non-temporal
// loads and write it back with non-temporal stores: the state is touched once per step, and with
// the state served from DRAM (B = 64, H = 16, D = 128) the step took 25.0 us this way against
// 29.0 us for cached accesses in column blocks.
template <int D, class T>
__global__ __launch_bounds__(256) void gated_delta_decode_w4_kernel(DecodeParams p) {
  constexpr int W = 4, VB = 32, NWB = D / VB;                // column blocks, one per wave (waves 0..NWB-1)
  constexpr int CG = VB / 4, RG = kWave / CG, RPT = D / RG;  // lane (rg, cg): rows rg + RG i, columns 4cg..+3
  using Win = ConvWindow<W, T>;
  __shared__ float qk[2 * D];
  __shared__ float vs[2][D];
  const int h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int rep = (int)(p.HV / p.H);
  const int64_t C = (2 * p.H + p.HV) * D;
  const int t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave, cg = lane % CG, rg = lane / CG;
  const T* __restrict__ xg = static_cast<const T*>(p.x);
  Win* __restrict__ cs = static_cast<Win*>(p.conv_state);
  const float4* __restrict__ wg = reinterpret_cast<const float4*>(p.conv_w);
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const bool has_qk = t < 2 * D, has_v = t < D;
  const int64_t ch_qk = (t < D) ? (int64_t)h * D + t : p.H * D + (int64_t)h * D + (t - D);

  for (int r = 0; r < rep; ++r) {
    const int hv = h * rep + r;
    const int par = r & 1;
    const int64_t sbase = (b * p.HV + hv) * (int64_t)D * D;
    const int64_t ch_v = 2 * p.H * D + (int64_t)hv * D + t;
    // The state first, so that the step's 64 KB per head is in flight before the conv window and
    // gate loads: through a buffer resource (one lane offset plus a scalar offset per row step, so
    // the 16 row addresses take no registers), non-temporal (the state is touched once a step).
    float4 s[RPT];
    const auto rs = make_rsrc(p.state + sbase, (uint32_t)(D * D * 4));
    const int voff = ((rg * D) + w * VB + 4 * cg) * 4;
    if (w < NWB) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, i * RG * D * 4, 2);
        s[i] = __builtin_bit_cast(float4, x);
      }
    }
    Win wq{}, wv{};
    T xq{}, xv{};
    float4 kq{}, kv{};
    const bool do_qk = has_qk && r == 0;
    if (do_qk) {
      wq = cs[b * C + ch_qk];
      xq = xg[b * C + ch_qk];
      kq = wg[ch_qk];
    }
    if (has_v) {
      wv = cs[b * C + ch_v];
      xv = xg[b * C + ch_v];
      kv = wg[ch_v];
    }
    const uint32_t graw = load_raw32(p.g, p.dg, b * p.HV + hv);
    const uint32_t braw = load_raw32(p.beta, p.db, b * p.HV + hv);
    if (do_qk) {
      const float y = kq.x * elem_to_f32(wq.v[1]) + kq.y * elem_to_f32(wq.v[2]) + kq.z * elem_to_f32(wq.v[3]) +
                      kq.w * elem_to_f32(xq);
      Win nw;
      nw.v[0] = wq.v[1]; nw.v[1] = wq.v[2]; nw.v[2] = wq.v[3]; nw.v[3] = xq;
      cs[b * C + ch_qk] = nw;
      qk[t] = elem_to_f32(f32_to_elem<T>(silu_f32(y)));
    }
    if (has_v) {
      const float y = kv.x * elem_to_f32(wv.v[1]) + kv.y * elem_to_f32(wv.v[2]) + kv.z * elem_to_f32(wv.v[3]) +
                      kv.w * elem_to_f32(xv);
      Win nw;
      nw.v[0] = wv.v[1]; nw.v[1] = wv.v[2]; nw.v[2] = wv.v[3]; nw.v[3] = xv;
      cs[b * C + ch_v] = nw;
      vs[par][t] = elem_to_f32(f32_to_elem<T>(silu_f32(y)));
    }
    float gv = raw32_to_f32(graw, p.dg), bv = raw32_to_f32(braw, p.db);
    if (p.flags & GDN_FLAG_GATE_IN_KERNEL) gv = -expf(p.A_log[hv]) * softplus_f32(gv + p.dt_bias[hv]);
    if (p.flags & GDN_FLAG_BETA_SIGMOID) bv = sigmoid_f32(bv);
    const float a = expf(gv);
    __syncthreads();
    if (w < NWB) {
      const float* q_l = qk;
      const float* k_l = qk + D;
      float pr[11];
#pragma unroll
      for (int j2 = 0; j2 < 11; ++j2) pr[j2] = 0.f;
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int row = rg + RG * i;
        const float kr = k_l[row], qr = q_l[row];
        pr[0] += s[i].x * kr; pr[1] += s[i].y * kr; pr[2] += s[i].z * kr; pr[3] += s[i].w * kr;
        pr[4] += s[i].x * qr; pr[5] += s[i].y * qr; pr[6] += s[i].z * qr; pr[7] += s[i].w * qr;
        pr[8] += kr * qr; pr[9] += kr * kr; pr[10] += qr * qr;
      }
#pragma unroll
      for (int j2 = 0; j2 < 11; ++j2) pr[j2] = rg_sum(pr[j2]);
      const float ik = l2 ? 1.f / fmaxf(sqrtf(pr[9]), 1e-12f) : 1.f;
      const float iq = l2 ? 1.f / fmaxf(sqrtf(pr[10]), 1e-12f) : 1.f;
      const float* v_l = vs[par] + w * VB + 4 * cg;
      float d[4], o4[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        d[c] = bv * (v_l[c] - a * pr[c] * ik);
        o4[c] = p.scale * (a * pr[4 + c] * iq + d[c] * pr[8] * ik * iq);
      }
      if (rg == 0) {
        T* og = static_cast<T*>(p.o) + (b * p.HV + hv) * D + w * VB + 4 * cg;
#pragma unroll
        for (int c = 0; c < 4; ++c) og[c] = f32_to_elem<T>(o4[c]);
      }
      // the row step goes into the lane offset, not the scalar offset: for a wide buffer store whose
      // scalar offset is a register the compiler inserts no wait states before the store's data
      // registers are rewritten, and the last lanes of a row then stored the rewritten values
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float kr = k_l[rg + RG * i] * ik;
        const float4 n{a * s[i].x + kr * d[0], a * s[i].y + kr * d[1], a * s[i].z + kr * d[2], a * s[i].w + kr * d[3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, n), rs, voff + i * RG * D * 4, 0, 2);
      }
    }
  }
}

}  // namespace gdn

using namespace gdn;

static int check_dims(int64_t K, int64_t V) {
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) {
    gdn_internal_set_error("head dims K=%lld V=%lld unsupported (each must be 64 or 128)", (long long)K, (long long)V);
    return GDN_ERR_UNSUPPORTED;
  }
  return GDN_OK;
}

extern "C" int gdn_recurrent_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                 const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                                 int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                                 int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                                 const float* A_log, const float* dt_bias, void* stream) {
  if (!q || !k || !v || !g || !beta || !o) {
    gdn_internal_set_error("gdn_recurrent_fwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || H <= 0 || HV <= 0 || HV % H || N <= 0) {
    gdn_internal_set_error("gdn_recurrent_fwd: bad sizes B=%lld T=%lld H=%lld HV=%lld N=%lld", (long long)B,
                           (long long)T, (long long)H, (long long)HV, (long long)N);
    return GDN_ERR_INVALID;
  }
  if (cu_seqlens ? B != 1 : N != B) {
    gdn_internal_set_error("gdn_recurrent_fwd: cu_seqlens requires B == 1 (and N == B without it)");
    return GDN_ERR_INVALID;
  }
  if ((flags & GDN_FLAG_GATE_IN_KERNEL) && (!A_log || !dt_bias)) {
    gdn_internal_set_error("gdn_recurrent_fwd: gate in kernel needs A_log and dt_bias");
    return GDN_ERR_INVALID;
  }
  if (int rc = check_dims(K, V)) return rc;
  if (N > 65535) {
    gdn_internal_set_error("gdn_recurrent_fwd: N=%lld exceeds the grid limit 65535", (long long)N);
    return GDN_ERR_UNSUPPORTED;
  }
  RecParams p{q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, (flags & GDN_FLAG_CU_INT32) ? 1 : 0,
              T, H, HV, qkv_dtype, g_dtype, beta_dtype, scale, flags, A_log, dt_bias};
  dim3 grid((unsigned)HV, (unsigned)N), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_recurrent_kernel<128, 128>), grid, block, 0, s, p);
  else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_recurrent_kernel<64, 64>), grid, block, 0, s, p);
  else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_recurrent_kernel<128, 64>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gated_delta_recurrent_kernel<64, 128>), grid, block, 0, s, p);
  return gdn_internal_check_launch("gated_delta_recurrent_kernel");
}

extern "C" int gdn_decode_step(const void* x_qkv, void* conv_state, const float* conv_weight, const void* g,
                               const void* beta, float* state, void* o, int64_t B, int64_t H, int64_t HV, int64_t D,
                               int64_t W, int x_dtype, int conv_state_dtype, int g_dtype, int beta_dtype, float scale,
                               unsigned flags, const float* A_log, const float* dt_bias, void* stream) {
  if (!x_qkv || !conv_state || !conv_weight || !g || !beta || !state || !o) {
    gdn_internal_set_error("gdn_decode_step: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || H <= 0 || HV <= 0 || HV % H || W < 1 || W > 16) {
    gdn_internal_set_error("gdn_decode_step: bad sizes B=%lld H=%lld HV=%lld W=%lld", (long long)B, (long long)H,
                           (long long)HV, (long long)W);
    return GDN_ERR_INVALID;
  }
  if (D != 64 && D != 128) {
    gdn_internal_set_error("gdn_decode_step: head dim %lld unsupported (64 or 128)", (long long)D);
    return GDN_ERR_UNSUPPORTED;
  }
  if ((flags & GDN_FLAG_GATE_IN_KERNEL) && (!A_log || !dt_bias)) {
    gdn_internal_set_error("gdn_decode_step: gate in kernel needs A_log and dt_bias");
    return GDN_ERR_INVALID;
  }
  if (B > 65535) {
    gdn_internal_set_error("gdn_decode_step: B=%lld exceeds the grid limit 65535", (long long)B);
    return GDN_ERR_UNSUPPORTED;
  }
  DecodeParams p{x_qkv, conv_state, conv_weight, g, beta, state, o, H, HV, W, x_dtype, conv_state_dtype,
                 g_dtype, beta_dtype, scale, flags, A_log, dt_bias};
  dim3 grid((unsigned)H, (unsigned)B), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (W == 4 && conv_state_dtype == x_dtype) {  // vectorised width-4 path
#define GDN_DECODE_W4(D_, T_) hipLaunchKernelGGL((gated_delta_decode_w4_kernel<D_, T_>), grid, block, 0, s, p)
    if (x_dtype == GDN_DTYPE_BF16) { if (D == 128) GDN_DECODE_W4(128, bf16); else GDN_DECODE_W4(64, bf16); }
    else if (x_dtype == GDN_DTYPE_F16) { if (D == 128) GDN_DECODE_W4(128, f16); else GDN_DECODE_W4(64, f16); }
    else { if (D == 128) GDN_DECODE_W4(128, float); else GDN_DECODE_W4(64, float); }
#undef GDN_DECODE_W4
    return gdn_internal_check_launch("gated_delta_decode_w4_kernel");
  }
  if (D == 128) hipLaunchKernelGGL((gated_delta_decode_kernel<128>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gated_delta_decode_kernel<64>), grid, block, 0, s, p);
  return gdn_internal_check_launch("gated_delta_decode_kernel");
}

// Depthwise causal conv1d (+ SiLU) with per-document reset: the q/k/v prologue of the GDN layer.
//
// y_t[c] = act(bias[c] + sum_j w[c, W-1-j] x_{t-j}[c]), with x_{t-j} taken as 0 (or from the
// initial conv state) when t-j lies before the start of t's document (sore/model/conv.py:6-23;
// a term from another document is never read, so a NaN there cannot leak, conv.py:18-21).
// One thread per channel walks TT consecutive tokens with the last W-1 inputs in registers; a
// wave covers 64 consecutive channels, so every load and store of a token row is coalesced.

#include <type_traits>

#include "gdn_common.h"

namespace gdn {

struct ConvParams {
  const void* x;
  const float* w;
  const float* bias;
  void* y;
  const void* init;
  void* fin;
  const void* cu;
  int cu_i32;
  int64_t T, C, N;
  int dx, act;
};

constexpr int kConvTokens = 64;

template <int W>
__global__ __launch_bounds__(256) void gated_delta_conv1d_kernel(ConvParams p) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= p.C) return;
  const int64_t bb = blockIdx.z;  // batch row (B == 1 with cu_seqlens)
  const int64_t t0 = (int64_t)blockIdx.y * kConvTokens;
  if (t0 >= p.T) return;
  const int64_t t1 = t0 + kConvTokens < p.T ? t0 + kConvTokens : p.T;
  float w[W];
#pragma unroll
  for (int i = 0; i < W; ++i) w[i] = p.w[c * W + i];
  const float bias = p.bias ? p.bias[c] : 0.f;

  // document containing t0
  int64_t d = bb, ds = 0, de = p.T;
  if (p.cu) {
    int64_t lo = 0, hi = p.N - 1;  // largest d with cu[d] <= t0
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (load_index(p.cu, p.cu_i32, mid) <= t0) lo = mid;
      else hi = mid - 1;
    }
    d = lo;
    ds = load_index(p.cu, p.cu_i32, d);
    de = load_index(p.cu, p.cu_i32, d + 1);
  }
  const int64_t row = bb * p.T;  // flat token offset of this batch row
  // win[i] holds the input at position t - (W-1) + i for the next token t
  float win[W > 1 ? W - 1 : 1];
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int64_t pos = t0 - (W - 1) + i;
    if (pos >= ds) win[i] = load_as_f32(p.x, p.dx, (row + pos) * p.C + c);
    else if (p.init) win[i] = load_as_f32(p.init, p.dx, (d * p.C + c) * W + (W - (ds - pos)));
    else win[i] = 0.f;
  }
  for (int64_t t = t0; t < t1; ++t) {
    while (t >= de) {  // next document: restart the window from its initial state
      ++d;
      ds = de;
      de = load_index(p.cu, p.cu_i32, d + 1);
#pragma unroll
      for (int i = 0; i < W - 1; ++i)
        win[i] = p.init ? load_as_f32(p.init, p.dx, (d * p.C + c) * W + i + 1) : 0.f;
    }
    const float xt = load_as_f32(p.x, p.dx, (row + t) * p.C + c);
    float acc = bias + w[W - 1] * xt;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) acc += w[i] * win[i];
    if (p.act == GDN_ACT_SILU) acc = silu_f32(acc);
    store_from_f32(p.y, p.dx, (row + t) * p.C + c, acc);
    const float dropped = W > 1 ? win[0] : xt;
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i) win[i] = win[i + 1];
    if (W > 1) win[W - 2] = xt;
    if (p.fin && t == de - 1) {  // last token of document d: the cache is its last W inputs
      const int64_t fb = (d * p.C + c) * W;
      if (W > 1) {
        store_from_f32(p.fin, p.dx, fb, dropped);
#pragma unroll
        for (int i = 0; i < W - 1; ++i) store_from_f32(p.fin, p.dx, fb + 1 + i, win[i]);
      } else {
        store_from_f32(p.fin, p.dx, fb, xt);
      }
    }
  }
}

// Vector path for 16-bit activations with C % 8 == 0: each thread owns 8 consecutive channels
// (16-byte loads and stores of a token row; a wave covers 512 channels, 1 KB per token) and walks
// kConvV8Tokens tokens, issuing the loads of 8 token rows before it uses the first. Same
// semantics and document handling as gated_delta_conv1d_kernel.
constexpr int kConvV8Tokens = 32;

template <int W, typename E>
__global__ __launch_bounds__(256) void gated_delta_conv1d_v8_kernel(ConvParams p) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  const int64_t c0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (c0 >= p.C) return;
  const int64_t bb = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * kConvV8Tokens;
  if (t0 >= p.T) return;
  const int64_t t1 = t0 + kConvV8Tokens < p.T ? t0 + kConvV8Tokens : p.T;
  const E* __restrict__ xs = static_cast<const E*>(p.x) + bb * p.T * p.C + c0;
  E* __restrict__ ys = static_cast<E*>(p.y) + bb * p.T * p.C + c0;
  const E* init = static_cast<const E*>(p.init);
  float w[8][W], bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int i = 0; i < W; ++i) w[e][i] = p.w[(c0 + e) * W + i];
    bias[e] = p.bias ? p.bias[c0 + e] : 0.f;
  }
  int64_t d = bb, ds = 0, de = p.T;
  if (p.cu) {
    int64_t lo = 0, hi = p.N - 1;  // largest d with cu[d] <= t0
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (load_index(p.cu, p.cu_i32, mid) <= t0) lo = mid;
      else hi = mid - 1;
    }
    d = lo;
    ds = load_index(p.cu, p.cu_i32, d);
    de = load_index(p.cu, p.cu_i32, d + 1);
  }
  // win[i][e]: input at position t - (W-1) + i of channel c0 + e for the next token t
  float win[W > 1 ? W - 1 : 1][8];
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int64_t pos = t0 - (W - 1) + i;
    if (pos >= ds) {
      const V8 v = *reinterpret_cast<const V8*>(xs + pos * p.C);
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = (float)v[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = init ? (float)init[(d * p.C + c0 + e) * W + (W - (ds - pos))] : 0.f;
    }
  }
  for (int64_t tg = t0; tg < t1; tg += 8) {
    V8 xv[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {  // rows past t1 re-read the last valid row (never used)
      const int64_t tt = tg + g < t1 ? tg + g : t1 - 1;
      xv[g] = *reinterpret_cast<const V8*>(xs + tt * p.C);
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int64_t t = tg + g;
      if (t >= t1) break;
      while (t >= de) {  // next document: restart the window from its initial state
        ++d;
        ds = de;
        de = load_index(p.cu, p.cu_i32, d + 1);
#pragma unroll
        for (int i = 0; i < W - 1; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) win[i][e] = init ? (float)init[(d * p.C + c0 + e) * W + i + 1] : 0.f;
      }
      V8 yv;
      float xt[8], dropped[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xt[e] = (float)xv[g][e];
        float acc = bias[e] + w[e][W - 1] * xt[e];
#pragma unroll
        for (int i = 0; i < W - 1; ++i) acc += w[e][i] * win[i][e];
        if (p.act == GDN_ACT_SILU) acc = silu_fast(acc);
        yv[e] = (E)acc;
        dropped[e] = W > 1 ? win[0][e] : xt[e];
#pragma unroll
        for (int i = 0; i + 1 < W - 1; ++i) win[i][e] = win[i + 1][e];
        if (W > 1) win[W - 2][e] = xt[e];
      }
      *reinterpret_cast<V8*>(ys + t * p.C) = yv;
      if (p.fin && t == de - 1) {  // last token of document d: the cache is its last W inputs
        E* fin = static_cast<E*>(p.fin);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t fb = (d * p.C + c0 + e) * W;
          if (W > 1) {
            fin[fb] = (E)dropped[e];
#pragma unroll
            for (int i = 0; i < W - 1; ++i) fin[fb + 1 + i] = (E)win[i][e];
          } else {
            fin[fb] = (E)xt[e];
          }
        }
      }
    }
  }
}

// The GDN layer's whole q/k/v prologue in one pass (inference): the packed projection output
// x [B, T, >= 2*Cqk + Cv] (row stride x_stride, e.g. the q|k|v columns of one fused GEMM output)
// -> depthwise causal conv (width 4) + SiLU, rounded to the activation dtype as the separate conv
// stores it, then, with l2, each q and k head of D channels L2-normalised (x / max(|x|, 1e-12) as
// v_rsq_f32 of max(|x|^2, 1e-24), the chunk kernels' in-kernel formula; fp32 math, rounded again)
// -> contiguous q, k [B, T, Cqk] and v [B, T, Cv].
// Thread = 8 channels as in gated_delta_conv1d_v8_kernel; a head of D channels is D/8 consecutive
// lanes, so its sum of squares is a DPP group sum. No conv caches (the layer's forward uses none).
// The activation and the varlen document walk are template parameters, so the unrolled row loop has
// no branches on them (with the reciprocal square root: 110 -> 104 us at config 4's shape).
struct QkvConvParams {
  const void* x;
  int64_t x_stride;
  const float* w;  // [2*Cqk + Cv][4]
  const float* bias;
  void *q, *k, *v;
  const void* cu;
  int cu_i32;
  int64_t T, Cqk, Cv, N;
  int act, l2;
};

template <typename E, int D, int ACT, bool VARLEN>
__global__ __launch_bounds__(256) void gated_delta_qkv_conv1d_kernel(QkvConvParams p) {
  constexpr int W = 4;
  typedef E V8 __attribute__((ext_vector_type(8)));
  const int64_t ctot = 2 * p.Cqk + p.Cv;
  const int64_t c0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  // threads past the channel count still run (clamped to the last chunk) so that every lane of a
  // head's group takes part in the group sum; only their stores are dropped
  const bool ch_ok = c0 < ctot;
  const int64_t cc = ch_ok ? c0 : ctot - 8;
  const int64_t bb = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * kConvV8Tokens;
  if (t0 >= p.T) return;
  const int64_t t1 = t0 + kConvV8Tokens < p.T ? t0 + kConvV8Tokens : p.T;
  const E* __restrict__ xs = static_cast<const E*>(p.x) + bb * p.T * p.x_stride + cc;
  // output and its channel offset: q | k | v
  E* dst;
  int64_t dc, dstride;
  if (cc < p.Cqk) {
    dst = static_cast<E*>(p.q); dc = cc; dstride = p.Cqk;
  } else if (cc < 2 * p.Cqk) {
    dst = static_cast<E*>(p.k); dc = cc - p.Cqk; dstride = p.Cqk;
  } else {
    dst = static_cast<E*>(p.v); dc = cc - 2 * p.Cqk; dstride = p.Cv;
  }
  E* __restrict__ ys = dst + bb * p.T * dstride + dc;
  const bool norm = p.l2 && cc < 2 * p.Cqk;  // uniform across a head's lanes (heads never straddle q|k|v)
  float w[8][W], bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int i = 0; i < W; ++i) w[e][i] = p.w[(cc + e) * W + i];
    bias[e] = p.bias ? p.bias[cc + e] : 0.f;
  }
  int64_t d = 0, ds = 0, de = p.T;
  if (VARLEN) {
    int64_t lo = 0, hi = p.N - 1;  // largest d with cu[d] <= t0
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (load_index(p.cu, p.cu_i32, mid) <= t0) lo = mid;
      else hi = mid - 1;
    }
    d = lo;
    ds = load_index(p.cu, p.cu_i32, d);
    de = load_index(p.cu, p.cu_i32, d + 1);
  }
  float win[W - 1][8];
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int64_t pos = t0 - (W - 1) + i;
    if (pos >= ds) {
      const V8 xv = *reinterpret_cast<const V8*>(xs + pos * p.x_stride);
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = (float)xv[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = 0.f;
    }
  }
  for (int64_t tg = t0; tg < t1; tg += 8) {
    V8 xv[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {  // rows past t1 re-read the last valid row (never used)
      const int64_t tt = tg + g < t1 ? tg + g : t1 - 1;
      xv[g] = *reinterpret_cast<const V8*>(xs + tt * p.x_stride);
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int64_t t = tg + g;
      if (t >= t1) break;  // uniform: t1 is the same for the whole block
      while (VARLEN && t >= de) {  // next document: the window restarts from zeros
        ++d;
        ds = de;
        de = load_index(p.cu, p.cu_i32, d + 1);
#pragma unroll
        for (int i = 0; i < W - 1; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) win[i][e] = 0.f;
      }
      float y[8], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xt = (float)xv[g][e];
        float acc = bias[e] + w[e][W - 1] * xt;
#pragma unroll
        for (int i = 0; i < W - 1; ++i) acc += w[e][i] * win[i][e];
        if (ACT == GDN_ACT_SILU) acc = silu_fast(acc);
        // the reference's unfused route (sore/model/gdn.py:208-209): the conv output is rounded to the
        // activation dtype before F.silu
        else if (ACT == GDN_ACT_SILU_ROUNDED) acc = silu_fast((float)(E)acc);
        y[e] = (float)(E)acc;  // the separate conv's stored value
        ss += y[e] * y[e];
#pragma unroll
        for (int i = 0; i + 1 < W - 1; ++i) win[i][e] = win[i + 1][e];
        win[W - 2][e] = xt;
      }
      ss = group_sum<D / 8>(ss);
      const float inv = norm ? __builtin_amdgcn_rsqf(fmaxf(ss, 1e-24f)) : 1.f;
      V8 yv;
#pragma unroll
      for (int e = 0; e < 8; ++e) yv[e] = (E)(norm ? y[e] * inv : y[e]);
      if (ch_ok) *reinterpret_cast<V8*>(ys + t * dstride) = yv;
    }
  }
}

// Backward (the reference trains through it: FLA causal_conv1d's backward, or autograd through
// sore/model/conv.py:6-23 + F.silu). With z_t = bias + sum_j w[W-1-j] x_{t-j} and dz_t = dy_t act'(z_t):
//   dx_s = sum_j w[W-1-j] dz_{s+j}   (s + j in s's document),
//   dw[W-1-j] = sum_t dz_t x_{t-j},  dbias = sum_t dz_t,
//   d initial_state[n, W-m] = sum over the first tokens t of document n of w[W-1-j] dz_t, t - j = start - m.
// Same walk as the forward (thread = channel, 64 tokens per block, the window of inputs in registers)
// over the block's tokens plus the W-1 that follow it; the dx of a position is final once the W
// tokens that read it are done (a ring of W pending sums). dw and dbias leave as per-block partial
// sums (reduced by gated_delta_conv1d_param_grad_kernel); the initial-state gradient is added with
// atomics (a document's first tokens can span two blocks).
struct ConvBwdParams {
  const void* x;
  const float* w;
  const float* bias;
  const void* dy;
  const void* init;
  const void* cu;
  int cu_i32;
  int64_t T, C, N;
  int dx_t, act;
  void* dx;
  float* part;   // [blocks][C][W + 1]
  float* dinit;  // [N][C][W] fp32, zeroed first, or null
};

template <int W>
__global__ __launch_bounds__(256) void gated_delta_conv1d_bwd_kernel(ConvBwdParams p) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= p.C) return;
  const int64_t bb = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * kConvTokens;
  if (t0 >= p.T) return;
  const int64_t t1 = t0 + kConvTokens < p.T ? t0 + kConvTokens : p.T;
  const int64_t tend = t1 + W - 1 < p.T ? t1 + W - 1 : p.T;
  float w[W];
#pragma unroll
  for (int i = 0; i < W; ++i) w[i] = p.w[c * W + i];
  const float bias = p.bias ? p.bias[c] : 0.f;
  int64_t d = bb, ds = 0, de = p.T;
  if (p.cu) {
    int64_t lo = 0, hi = p.N - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (load_index(p.cu, p.cu_i32, mid) <= t0) lo = mid;
      else hi = mid - 1;
    }
    d = lo;
    ds = load_index(p.cu, p.cu_i32, d);
    de = load_index(p.cu, p.cu_i32, d + 1);
  }
  const int64_t row = bb * p.T;
  float win[W > 1 ? W - 1 : 1];  // inputs at t - (W-1) + i
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int64_t pos = t0 - (W - 1) + i;
    if (pos >= ds) win[i] = load_as_f32(p.x, p.dx_t, (row + pos) * p.C + c);
    else if (p.init) win[i] = load_as_f32(p.init, p.dx_t, (d * p.C + c) * W + (W - (ds - pos)));
    else win[i] = 0.f;
  }
  float pend[W];  // pending dx of positions t - (W-1) + i
#pragma unroll
  for (int i = 0; i < W; ++i) pend[i] = 0.f;
  float dw[W], db = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) dw[i] = 0.f;
  for (int64_t t = t0; t < tend; ++t) {
    // position t - W is complete: store it if this block owns it
    if (t - W >= t0) store_from_f32(p.dx, p.dx_t, (row + t - W) * p.C + c, pend[0]);
#pragma unroll
    for (int i = 0; i + 1 < W; ++i) pend[i] = pend[i + 1];
    pend[W - 1] = 0.f;
    while (t >= de) {
      ++d;
      ds = de;
      de = load_index(p.cu, p.cu_i32, d + 1);
#pragma unroll
      for (int i = 0; i < W - 1; ++i)
        win[i] = p.init ? load_as_f32(p.init, p.dx_t, (d * p.C + c) * W + i + 1) : 0.f;
    }
    const float xt = load_as_f32(p.x, p.dx_t, (row + t) * p.C + c);
    float z = bias + w[W - 1] * xt;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) z += w[i] * win[i];
    float dz = load_as_f32(p.dy, p.dx_t, (row + t) * p.C + c);
    if (p.act == GDN_ACT_SILU) {
      const float sg = sigmoid_f32(z);
      dz *= sg * (1.f + z * (1.f - sg));
    }
    const bool own = t < t1;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int64_t pos = t - j;
      const float xin = j == 0 ? xt : win[W - 1 - j];
      if (pos >= ds) {
        pend[W - 1 - j] += w[W - 1 - j] * dz;
      } else if (own && p.dinit) {
        atomicAdd(&p.dinit[(d * p.C + c) * W + (W - (ds - pos))], w[W - 1 - j] * dz);
      }
      if (own) dw[W - 1 - j] += dz * xin;
    }
    if (own) db += dz;
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i) win[i] = win[i + 1];
    if (W > 1) win[W - 2] = xt;
  }
  // flush: pend[i] is position tend - W + i
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const int64_t pos = tend - W + i;
    if (pos >= t0 && pos < t1) store_from_f32(p.dx, p.dx_t, (row + pos) * p.C + c, pend[i]);
  }
  const int64_t blk = bb * gridDim.y + blockIdx.y;
  float* pp = p.part + (blk * p.C + c) * (W + 1);
#pragma unroll
  for (int i = 0; i < W; ++i) pp[i] = dw[i];
  pp[W] = db;
}

// dweight [C][W] and dbias [C] (fp32) from the per-block partial sums [blocks][C][W + 1].
__global__ __launch_bounds__(256) void gated_delta_conv1d_param_grad_kernel(const float* part, int64_t blocks, int64_t C,
                                                                            int W, float* dw, float* dbias) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // = c * (W + 1) + i
  if (e >= C * (W + 1)) return;
  float acc = 0.f;
  for (int64_t b = 0; b < blocks; ++b) acc += part[b * C * (W + 1) + e];
  const int64_t c = e / (W + 1), i = e % (W + 1);
  if (i < W) dw[c * W + i] = acc;
  else if (dbias) dbias[c] = acc;
}

__global__ void gated_delta_fill_zero_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_causal_conv1d_fwd(const void* x, const float* weight, const float* bias, void* y,
                                     const void* initial_state, void* final_state, const void* cu_seqlens, int64_t B,
                                     int64_t T, int64_t C, int64_t W, int64_t N, int x_dtype, int activation,
                                     unsigned flags, void* stream) {
  if (!x || !weight || !y) {
    gdn_internal_set_error("gdn_causal_conv1d_fwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || C <= 0 || N <= 0 || (cu_seqlens ? B != 1 : N != B)) {
    gdn_internal_set_error("gdn_causal_conv1d_fwd: bad sizes B=%lld T=%lld C=%lld N=%lld (cu_seqlens needs B == 1)",
                           (long long)B, (long long)T, (long long)C, (long long)N);
    return GDN_ERR_INVALID;
  }
  if (W < 1 || W > 8) {
    gdn_internal_set_error("gdn_causal_conv1d_fwd: kernel width %lld unsupported (1..8)", (long long)W);
    return GDN_ERR_UNSUPPORTED;
  }
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU) {
    gdn_internal_set_error("gdn_causal_conv1d_fwd: unknown activation %d", activation);
    return GDN_ERR_INVALID;
  }
  if (T == 0) return GDN_OK;
  const int64_t tb = (T + kConvTokens - 1) / kConvTokens;
  if (tb > 65535 || B > 65535) {
    gdn_internal_set_error("gdn_causal_conv1d_fwd: T=%lld B=%lld exceed the grid limits", (long long)T, (long long)B);
    return GDN_ERR_UNSUPPORTED;
  }
  ConvParams p{x, weight, bias, y, initial_state, final_state, cu_seqlens, (flags & GDN_FLAG_CU_INT32) ? 1 : 0,
               T, C, N, x_dtype, activation};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tb8 = (T + kConvV8Tokens - 1) / kConvV8Tokens;
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  if (aligned && C % 8 == 0 && W == 4 && tb8 <= 65535 && (x_dtype == GDN_DTYPE_BF16 || x_dtype == GDN_DTYPE_F16)) {
    const dim3 g8((unsigned)((C / 8 + 255) / 256), (unsigned)tb8, (unsigned)B), b8(256);
    if (x_dtype == GDN_DTYPE_BF16) hipLaunchKernelGGL((gated_delta_conv1d_v8_kernel<4, bf16>), g8, b8, 0, s, p);
    else hipLaunchKernelGGL((gated_delta_conv1d_v8_kernel<4, f16>), g8, b8, 0, s, p);
    return gdn_internal_check_launch("gated_delta_conv1d_v8_kernel");
  }
  dim3 grid((unsigned)((C + 255) / 256), (unsigned)tb, (unsigned)B), block(256);
  switch (W) {
    case 1: hipLaunchKernelGGL(gated_delta_conv1d_kernel<1>, grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL(gated_delta_conv1d_kernel<2>, grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL(gated_delta_conv1d_kernel<3>, grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL(gated_delta_conv1d_kernel<4>, grid, block, 0, s, p); break;
    case 5: hipLaunchKernelGGL(gated_delta_conv1d_kernel<5>, grid, block, 0, s, p); break;
    case 6: hipLaunchKernelGGL(gated_delta_conv1d_kernel<6>, grid, block, 0, s, p); break;
    case 7: hipLaunchKernelGGL(gated_delta_conv1d_kernel<7>, grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL(gated_delta_conv1d_kernel<8>, grid, block, 0, s, p); break;
  }
  return gdn_internal_check_launch("gated_delta_conv1d_kernel");
}

extern "C" size_t gdn_causal_conv1d_bwd_workspace_size(int64_t B, int64_t T, int64_t C, int64_t W) {
  if (B <= 0 || T < 0 || C <= 0 || W < 1) return 0;
  return (size_t)(B * ((T + kConvTokens - 1) / kConvTokens) * C * (W + 1) * 4);
}

extern "C" int gdn_causal_conv1d_bwd(const void* x, const float* weight, const float* bias, const void* dy,
                                     const void* initial_state, const void* cu_seqlens, int64_t B, int64_t T, int64_t C,
                                     int64_t W, int64_t N, int x_dtype, int activation, unsigned flags, void* dx,
                                     float* dweight, float* dbias, float* d_initial_state, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (!x || !weight || !dy || !dx || !dweight) {
    gdn_internal_set_error("gdn_causal_conv1d_bwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || C <= 0 || N <= 0 || (cu_seqlens ? B != 1 : N != B)) {
    gdn_internal_set_error("gdn_causal_conv1d_bwd: bad sizes B=%lld T=%lld C=%lld N=%lld (cu_seqlens needs B == 1)",
                           (long long)B, (long long)T, (long long)C, (long long)N);
    return GDN_ERR_INVALID;
  }
  if (W < 1 || W > 8) {
    gdn_internal_set_error("gdn_causal_conv1d_bwd: kernel width %lld unsupported (1..8)", (long long)W);
    return GDN_ERR_UNSUPPORTED;
  }
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU) {
    gdn_internal_set_error("gdn_causal_conv1d_bwd: unknown activation %d", activation);
    return GDN_ERR_INVALID;
  }
  const size_t need = gdn_causal_conv1d_bwd_workspace_size(B, T, C, W);
  if (need > 0 && (!workspace || workspace_bytes < need)) {
    gdn_internal_set_error("gdn_causal_conv1d_bwd: workspace of %zu bytes needed", need);
    return GDN_ERR_INVALID;
  }
  const int64_t tb = (T + kConvTokens - 1) / kConvTokens;
  if (tb > 65535 || B > 65535) {
    gdn_internal_set_error("gdn_causal_conv1d_bwd: T=%lld B=%lld exceed the grid limits", (long long)T, (long long)B);
    return GDN_ERR_UNSUPPORTED;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d_initial_state) {
    const int64_t n = N * C * W;
    hipLaunchKernelGGL(gated_delta_fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_initial_state, n);
  }
  if (T == 0) {
    const int64_t n = C * W;  // no tokens: zero parameter gradients
    hipLaunchKernelGGL(gated_delta_fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dweight, n);
    if (dbias) hipLaunchKernelGGL(gated_delta_fill_zero_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s, dbias, C);
    return gdn_internal_check_launch("gated_delta_fill_zero_kernel");
  }
  ConvBwdParams p{x, weight, bias, dy, initial_state, cu_seqlens, (flags & GDN_FLAG_CU_INT32) ? 1 : 0, T, C, N,
                  x_dtype, activation, dx, static_cast<float*>(workspace), initial_state ? d_initial_state : nullptr};
  dim3 grid((unsigned)((C + 255) / 256), (unsigned)tb, (unsigned)B), block(256);
  switch (W) {
    case 1: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<1>, grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<2>, grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<3>, grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<4>, grid, block, 0, s, p); break;
    case 5: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<5>, grid, block, 0, s, p); break;
    case 6: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<6>, grid, block, 0, s, p); break;
    case 7: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<7>, grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL(gated_delta_conv1d_bwd_kernel<8>, grid, block, 0, s, p); break;
  }
  int rc = gdn_internal_check_launch("gated_delta_conv1d_bwd_kernel");
  if (rc != GDN_OK) return rc;
  const int64_t ne = C * (W + 1);
  hipLaunchKernelGGL(gated_delta_conv1d_param_grad_kernel, dim3((unsigned)((ne + 255) / 256)), dim3(256), 0, s,
                     static_cast<const float*>(workspace), B * tb, C, (int)W, dweight, dbias);
  return gdn_internal_check_launch("gated_delta_conv1d_param_grad_kernel");
}

extern "C" int gdn_qkv_conv_fwd(const void* x, int64_t x_row_stride, const float* weight, const float* bias, void* q,
                                void* k, void* v, const void* cu_seqlens, int64_t B, int64_t T, int64_t Cqk,
                                int64_t Cv, int64_t head_dim, int64_t N, int x_dtype, int activation,
                                unsigned flags, void* stream) {
  if (!x || !weight || !q || !k || !v) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || Cqk <= 0 || Cv <= 0 || N <= 0 || (cu_seqlens ? B != 1 : N != B)) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: bad sizes B=%lld T=%lld Cqk=%lld Cv=%lld N=%lld (cu_seqlens needs B == 1)",
                           (long long)B, (long long)T, (long long)Cqk, (long long)Cv, (long long)N);
    return GDN_ERR_INVALID;
  }
  if ((head_dim != 64 && head_dim != 128) || Cqk % head_dim || Cv % head_dim) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: head_dim %lld unsupported (64 or 128, dividing Cqk and Cv)",
                           (long long)head_dim);
    return GDN_ERR_UNSUPPORTED;
  }
  if (x_dtype != GDN_DTYPE_BF16 && x_dtype != GDN_DTYPE_F16) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: activation dtype %d unsupported (bf16 or fp16)", x_dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU && activation != GDN_ACT_SILU_ROUNDED) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: unknown activation %d", activation);
    return GDN_ERR_INVALID;
  }
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q) |
                       reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v);
  if (x_row_stride < 2 * Cqk + Cv || x_row_stride % 8 || (al & 15)) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: x row stride %lld too small or buffers not 16-byte aligned",
                           (long long)x_row_stride);
    return GDN_ERR_INVALID;
  }
  if (T == 0) return GDN_OK;
  const int64_t tb = (T + kConvV8Tokens - 1) / kConvV8Tokens;
  if (tb > 65535 || B > 65535) {
    gdn_internal_set_error("gdn_qkv_conv_fwd: T=%lld B=%lld exceed the grid limits", (long long)T, (long long)B);
    return GDN_ERR_UNSUPPORTED;
  }
  QkvConvParams p{x, x_row_stride, weight, bias, q, k, v, cu_seqlens, (flags & GDN_FLAG_CU_INT32) ? 1 : 0, T, Cqk, Cv,
                  N, activation, (flags & GDN_FLAG_QK_L2NORM) ? 1 : 0};
  const int64_t threads = (2 * Cqk + Cv) / 8;
  const dim3 grid((unsigned)((threads + 255) / 256), (unsigned)tb, (unsigned)B), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // dtype, head dim, activation and varlen as template arguments
  auto go = [&](auto e_tag, auto d_c, auto a_c, auto v_c) {
    using E = decltype(e_tag);
    hipLaunchKernelGGL((gated_delta_qkv_conv1d_kernel<E, decltype(d_c)::value, decltype(a_c)::value, decltype(v_c)::value>),
                       grid, block, 0, s, p);
  };
  auto by_act = [&](auto e_tag, auto d_c, auto v_c) {
    if (activation == GDN_ACT_SILU) go(e_tag, d_c, std::integral_constant<int, GDN_ACT_SILU>{}, v_c);
    else if (activation == GDN_ACT_SILU_ROUNDED) go(e_tag, d_c, std::integral_constant<int, GDN_ACT_SILU_ROUNDED>{}, v_c);
    else go(e_tag, d_c, std::integral_constant<int, GDN_ACT_NONE>{}, v_c);
  };
  auto by_var = [&](auto e_tag, auto d_c) {
    if (cu_seqlens) by_act(e_tag, d_c, std::true_type{});
    else by_act(e_tag, d_c, std::false_type{});
  };
  auto by_d = [&](auto e_tag) {
    if (head_dim == 128) by_var(e_tag, std::integral_constant<int, 128>{});
    else by_var(e_tag, std::integral_constant<int, 64>{});
  };
  if (x_dtype == GDN_DTYPE_BF16) by_d(bf16{});
  else by_d(f16{});
  return gdn_internal_check_launch("gated_delta_qkv_conv1d_kernel");
}

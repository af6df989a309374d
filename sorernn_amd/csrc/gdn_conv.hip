// Depthwise causal conv1d (+ SiLU) with per-document reset: the q/k/v prologue of the GDN layer.
//
// y_t[c] = act(bias[c] + sum_j w[c, W-1-j] x_{t-j}[c]), with x_{t-j} taken as 0 (or from the
// initial conv state) when t-j lies before the start of t's document (sore/model/conv.py:6-23;
// a term from another document is never read, so a NaN there cannot leak, conv.py:18-21).
// One thread per channel walks TT consecutive tokens with the last W-1 inputs in registers; a
// wave covers 64 consecutive channels, so every load and store of a token row is coalesced.

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
  dim3 grid((unsigned)((C + 255) / 256), (unsigned)tb, (unsigned)B), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
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

// Row-wise epilogue/prologue norms: L2 normalisation (q/k) and gated RMSNorm (GDN output).
//
// One wave per row (rows of D = 64 or 128 elements in the GDN path, any D here): each lane reads
// D/64 elements, the sum of squares is reduced across the wave, and the row is written once with
// fp32 math and a single rounding. Both kernels are HBM-bound elementwise passes.

#include "gdn_chunk.h"

namespace gdn {

struct NormParams {
  const void* x;
  const void* gate;
  const float* w;
  const float* bias;
  void* y;
  int64_t rows, D;
  int dt, act;
  float eps;
  int mode;   // 0 = L2 norm, 1 = (gated) RMSNorm
  int split;  // RMSNorm with a gate: the norm (w, bias) and act(gate) each rounded before their product
};

constexpr int kNormMaxPerLane = 16;  // D <= 1024

__global__ __launch_bounds__(256) void gated_delta_norm_kernel(NormParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
  for (int64_t r = wave; r < p.rows; r += nwaves) {
    const int64_t base = r * p.D;
    float xv[kNormMaxPerLane];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormMaxPerLane; ++j) {
      const int64_t e = lane + (int64_t)j * kWave;
      xv[j] = e < p.D ? load_as_f32(p.x, p.dt, base + e) : 0.f;
      ss += xv[j] * xv[j];
    }
    ss = wave_xor_sum(ss, 1);
    float scale;
    if (p.mode == 0) scale = 1.f / fmaxf(sqrtf(ss), p.eps);  // F.normalize: x / max(||x||, eps)
    else scale = 1.f / sqrtf(ss / (float)p.D + p.eps);  // RMSNorm: rsqrt(mean(x^2) + eps)
#pragma unroll
    for (int j = 0; j < kNormMaxPerLane; ++j) {
      const int64_t e = lane + (int64_t)j * kWave;
      if (e >= p.D) break;
      float out = xv[j] * scale;
      if (p.mode == 1) {
        if (p.w) out *= p.w[e];
        if (p.bias) out += p.bias[e];
        if (p.gate) {
          const float gv = load_as_f32(p.gate, p.dt, base + e);
          const float a = (p.act == GDN_ACT_SILU) ? silu_f32(gv) : gv;
          out = p.split ? round_to(p.dt, out) * round_to(p.dt, a) : out * a;
        }
      }
      store_from_f32(p.y, p.dt, base + e, out);
    }
  }
}

// Vector path of the same two norms for 16-bit rows of D = 64 or 128: LPR = D / 8 lanes per row,
// each lane one 16-byte chunk of x (and of the gate), so a wave covers 64 / LPR rows with
// 16-byte loads and stores; the sum of squares is reduced inside the row's lane group by DPP.
// Each wave takes kNormV8Groups row groups per pass and issues all their loads before the first
// use (memory-level parallelism for an HBM-bound pass). fp32 math, one rounding; the RMS factor is
// v_rsq_f32 (the reference computes it with torch.rsqrt).
constexpr int kNormV8Groups = 4;

template <typename E, int LPR>
__global__ __launch_bounds__(256) void gated_delta_norm_v8_kernel(NormParams p) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  constexpr int RPW = kWave / LPR, U = kNormV8Groups;
  const int lane = threadIdx.x % kWave, sub = lane / LPR, li = lane % LPR;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
  const bool gated = p.mode == 1 && p.gate;
  float wv[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wv[e] = (p.mode == 1 && p.w) ? p.w[li * 8 + e] : 1.f;
    bv[e] = (p.mode == 1 && p.bias) ? p.bias[li * 8 + e] : 0.f;
  }
  for (int64_t r0 = wave * RPW * U; r0 < p.rows; r0 += nwaves * RPW * U) {
    V8 xv[U], gv[U];
    int64_t base[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {  // every lane loads (clamped rows): the reductions need all lanes
      const int64_t r = r0 + u * RPW + sub;
      base[u] = (r < p.rows ? r : p.rows - 1) * p.D + li * 8;
      xv[u] = *reinterpret_cast<const V8*>(static_cast<const E*>(p.x) + base[u]);
      if (gated) gv[u] = *reinterpret_cast<const V8*>(static_cast<const E*>(p.gate) + base[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float xf[8], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xf[e] = (float)xv[u][e];
        ss += xf[e] * xf[e];
      }
      ss = group_sum<LPR>(ss);
      const float scale = p.mode == 0 ? 1.f / fmaxf(sqrtf(ss), p.eps) : __builtin_amdgcn_rsqf(ss / (float)p.D + p.eps);
      V8 yv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float out = xf[e] * scale;
        if (p.mode == 1) {
          out = out * wv[e] + bv[e];
          if (gated) {
            const float g = (float)gv[u][e];
            const float a = (p.act == GDN_ACT_SILU) ? silu_fast(g) : g;
            out = p.split ? (float)(E)out * (float)(E)a : out * a;
          }
        }
        yv[e] = (E)out;
      }
      if (r0 + u * RPW + sub < p.rows) *reinterpret_cast<V8*>(static_cast<E*>(p.y) + base[u]) = yv;
    }
  }
}

// Backward of both norms, one wave per row (the reference trains through F.normalize and through
// RMSNorm * silu(gate) by autograd, sore/model/gdn.py:177,180-188; FLA's fused l2norm and
// rms_norm_gated kernels have their own backward):
//   L2:  y = x / max(|x|, eps):          dx = (dy - y (y . dy)) / |x|   (dy / eps where |x| <= eps)
//   RMS: n = x r, r = rsqrt(mean(x^2) + eps), u = n w + b, y = u act(g):
//        du = dy act(g), dg = dy u act'(g), dx = r (du w) - x r^3 mean((du w) x),
//        dw = sum_rows du n, db = sum_rows du  (per-wave partial sums, reduced by a second kernel).
struct NormBwdParams {
  const void* x;
  const void* gate;
  const float* w;
  const float* bias;
  const void* dy;
  void* dx;
  void* dgate;
  float* part;  // [waves][2][D] partial dw, db (RMS mode)
  int64_t rows, D;
  int dt, act;
  float eps;
  int mode;
};

__global__ __launch_bounds__(256) void gated_delta_norm_bwd_kernel(NormBwdParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
  float pw[kNormMaxPerLane], pb[kNormMaxPerLane];
#pragma unroll
  for (int j = 0; j < kNormMaxPerLane; ++j) pw[j] = pb[j] = 0.f;
  for (int64_t r = wave; r < p.rows; r += nwaves) {
    const int64_t base = r * p.D;
    float xv[kNormMaxPerLane], dv[kNormMaxPerLane];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormMaxPerLane; ++j) {
      const int64_t e = lane + (int64_t)j * kWave;
      xv[j] = e < p.D ? load_as_f32(p.x, p.dt, base + e) : 0.f;
      dv[j] = e < p.D ? load_as_f32(p.dy, p.dt, base + e) : 0.f;
      ss += xv[j] * xv[j];
    }
    ss = wave_xor_sum(ss, 1);
    if (p.mode == 0) {
      const float nrm = sqrtf(ss), inv = 1.f / fmaxf(nrm, p.eps);
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < kNormMaxPerLane; ++j) dot += xv[j] * inv * dv[j];
      dot = nrm > p.eps ? wave_xor_sum(dot, 1) : 0.f;
#pragma unroll
      for (int j = 0; j < kNormMaxPerLane; ++j) {
        const int64_t e = lane + (int64_t)j * kWave;
        if (e >= p.D) continue;
        store_from_f32(p.dx, p.dt, base + e, (dv[j] - xv[j] * inv * dot) * inv);
      }
    } else {
      const float rr = 1.f / sqrtf(ss / (float)p.D + p.eps);
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < kNormMaxPerLane; ++j) {
        const int64_t e = lane + (int64_t)j * kWave;
        if (e >= p.D) continue;
        const float n = xv[j] * rr, wv = p.w ? p.w[e] : 1.f;
        float du = dv[j];
        if (p.gate) {
          const float gv = load_as_f32(p.gate, p.dt, base + e);
          const float u = n * wv + (p.bias ? p.bias[e] : 0.f);
          float act = gv, dact = 1.f;
          if (p.act == GDN_ACT_SILU) {
            const float sg = sigmoid_f32(gv);
            act = gv * sg;
            dact = sg * (1.f + gv * (1.f - sg));
          }
          store_from_f32(p.dgate, p.dt, base + e, du * u * dact);
          du *= act;
        }
        pw[j] += du * n;
        pb[j] += du;
        dv[j] = du * wv;  // dn
        dot += dv[j] * xv[j];
      }
      dot = wave_xor_sum(dot, 1) / (float)p.D;
#pragma unroll
      for (int j = 0; j < kNormMaxPerLane; ++j) {
        const int64_t e = lane + (int64_t)j * kWave;
        if (e >= p.D) continue;
        store_from_f32(p.dx, p.dt, base + e, rr * dv[j] - xv[j] * rr * rr * rr * dot);
      }
    }
  }
  if (p.mode == 1) {
#pragma unroll
    for (int j = 0; j < kNormMaxPerLane; ++j) {
      const int64_t e = lane + (int64_t)j * kWave;
      if (e >= p.D) continue;
      p.part[(wave * 2) * p.D + e] = pw[j];
      p.part[(wave * 2 + 1) * p.D + e] = pb[j];
    }
  }
}

// dweight, dbias [D] from the per-wave partial sums [waves][2][D].
__global__ __launch_bounds__(256) void gated_delta_norm_param_grad_kernel(const float* part, int64_t waves, int64_t D,
                                                                          float* dw, float* db) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // = k * D + col, k = 0 (dw), 1 (db)
  if (e >= 2 * D) return;
  const int64_t k = e / D, col = e % D;
  float acc = 0.f;
  for (int64_t wv = 0; wv < waves; ++wv) acc += part[(wv * 2 + k) * D + col];
  float* out = k == 0 ? dw : db;
  if (out) out[col] = acc;
}

constexpr int64_t kNormBwdBlocks = 1024;  // the RMS backward's grid: 4096 waves of partial sums

static int launch_norm(const NormParams& p, void* stream, const char* what) {
  if (p.rows == 0) return GDN_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool aligned = ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.y) |
                         reinterpret_cast<uintptr_t>(p.gate)) & 15) == 0;
  if (aligned && (p.D == 64 || p.D == 128) && (p.dt == GDN_DTYPE_BF16 || p.dt == GDN_DTYPE_F16)) {
    const int64_t rpb = 4 * (kWave / (p.D / 8)) * kNormV8Groups;  // rows per 256-thread block and pass
    int64_t vb = (p.rows + rpb - 1) / rpb;
    if (vb > 65536) vb = 65536;
    const dim3 g((unsigned)vb), b(256);
    if (p.dt == GDN_DTYPE_BF16) {
      if (p.D == 128) hipLaunchKernelGGL((gated_delta_norm_v8_kernel<bf16, 16>), g, b, 0, s, p);
      else hipLaunchKernelGGL((gated_delta_norm_v8_kernel<bf16, 8>), g, b, 0, s, p);
    } else {
      if (p.D == 128) hipLaunchKernelGGL((gated_delta_norm_v8_kernel<f16, 16>), g, b, 0, s, p);
      else hipLaunchKernelGGL((gated_delta_norm_v8_kernel<f16, 8>), g, b, 0, s, p);
    }
    return gdn_internal_check_launch(what);
  }
  int64_t blocks = (p.rows + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(gated_delta_norm_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
  return gdn_internal_check_launch(what);
}

}  // namespace gdn

using namespace gdn;

int gdn::gdn_internal_rms_norm_gated(const void* x, const void* gate, const float* w, void* y, int64_t rows, int64_t D,
                                     float eps, int split, hipStream_t s) {
  NormParams p{x, gate, w, nullptr, y, rows, D, GDN_DTYPE_BF16, GDN_ACT_SILU, eps, 1, split};
  return launch_norm(p, s, "gated_delta_norm_kernel(rms)");
}

extern "C" int gdn_l2norm_fwd(const void* x, void* y, int64_t rows, int64_t D, int dtype, float eps, void* stream) {
  if (!x || !y || rows < 0 || D <= 0) {
    gdn_internal_set_error("gdn_l2norm_fwd: bad arguments (rows=%lld D=%lld)", (long long)rows, (long long)D);
    return GDN_ERR_INVALID;
  }
  if (D > kNormMaxPerLane * kWave) {
    gdn_internal_set_error("gdn_l2norm_fwd: D=%lld exceeds %d", (long long)D, kNormMaxPerLane * kWave);
    return GDN_ERR_UNSUPPORTED;
  }
  NormParams p{x, nullptr, nullptr, nullptr, y, rows, D, dtype, GDN_ACT_NONE, eps, 0};
  return launch_norm(p, stream, "gated_delta_norm_kernel(l2)");
}

extern "C" int gdn_rms_norm_gated_fwd(const void* x, const void* gate, const float* weight, const float* bias, void* y,
                                      int64_t rows, int64_t D, int dtype, float eps, int activation, void* stream) {
  if (!x || !y || rows < 0 || D <= 0) {
    gdn_internal_set_error("gdn_rms_norm_gated_fwd: bad arguments (rows=%lld D=%lld)", (long long)rows, (long long)D);
    return GDN_ERR_INVALID;
  }
  if (D > kNormMaxPerLane * kWave) {
    gdn_internal_set_error("gdn_rms_norm_gated_fwd: D=%lld exceeds %d", (long long)D, kNormMaxPerLane * kWave);
    return GDN_ERR_UNSUPPORTED;
  }
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU) {
    gdn_internal_set_error("gdn_rms_norm_gated_fwd: unknown activation %d", activation);
    return GDN_ERR_INVALID;
  }
  NormParams p{x, gate, weight, bias, y, rows, D, dtype, activation, eps, 1};
  return launch_norm(p, stream, "gated_delta_norm_kernel(rms)");
}

extern "C" int gdn_l2norm_bwd(const void* x, const void* dy, void* dx, int64_t rows, int64_t D, int dtype, float eps,
                              void* stream) {
  if (!x || !dy || !dx || rows < 0 || D <= 0) {
    gdn_internal_set_error("gdn_l2norm_bwd: bad arguments (rows=%lld D=%lld)", (long long)rows, (long long)D);
    return GDN_ERR_INVALID;
  }
  if (D > kNormMaxPerLane * kWave) {
    gdn_internal_set_error("gdn_l2norm_bwd: D=%lld exceeds %d", (long long)D, kNormMaxPerLane * kWave);
    return GDN_ERR_UNSUPPORTED;
  }
  if (rows == 0) return GDN_OK;
  NormBwdParams p{x, nullptr, nullptr, nullptr, dy, dx, nullptr, nullptr, rows, D, dtype, GDN_ACT_NONE, eps, 0};
  int64_t blocks = (rows + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(gated_delta_norm_bwd_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  return gdn_internal_check_launch("gated_delta_norm_bwd_kernel(l2)");
}

extern "C" size_t gdn_rms_norm_gated_bwd_workspace_size(int64_t rows, int64_t D) {
  if (rows < 0 || D <= 0) return 0;
  return (size_t)(kNormBwdBlocks * 4 * 2 * D * 4);
}

extern "C" int gdn_rms_norm_gated_bwd(const void* x, const void* gate, const float* weight, const float* bias,
                                      const void* dy, void* dx, void* dgate, float* dweight, float* dbias, int64_t rows,
                                      int64_t D, int dtype, float eps, int activation, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (!x || !dy || !dx || rows < 0 || D <= 0 || (gate && !dgate)) {
    gdn_internal_set_error("gdn_rms_norm_gated_bwd: bad arguments (rows=%lld D=%lld)", (long long)rows, (long long)D);
    return GDN_ERR_INVALID;
  }
  if (D > kNormMaxPerLane * kWave) {
    gdn_internal_set_error("gdn_rms_norm_gated_bwd: D=%lld exceeds %d", (long long)D, kNormMaxPerLane * kWave);
    return GDN_ERR_UNSUPPORTED;
  }
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU) {
    gdn_internal_set_error("gdn_rms_norm_gated_bwd: unknown activation %d", activation);
    return GDN_ERR_INVALID;
  }
  const size_t need = gdn_rms_norm_gated_bwd_workspace_size(rows, D);
  if (!workspace || workspace_bytes < need) {
    gdn_internal_set_error("gdn_rms_norm_gated_bwd: workspace of %zu bytes needed", need);
    return GDN_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  NormBwdParams p{x, gate, weight, bias, dy, dx, dgate, static_cast<float*>(workspace), rows, D, dtype, activation, eps, 1};
  hipLaunchKernelGGL(gated_delta_norm_bwd_kernel, dim3((unsigned)kNormBwdBlocks), dim3(256), 0, s, p);
  int rc = gdn_internal_check_launch("gated_delta_norm_bwd_kernel(rms)");
  if (rc != GDN_OK) return rc;
  hipLaunchKernelGGL(gated_delta_norm_param_grad_kernel, dim3((unsigned)((2 * D + 255) / 256)), dim3(256), 0, s,
                     static_cast<const float*>(workspace), (int64_t)kNormBwdBlocks * 4, D, dweight, dbias);
  return gdn_internal_check_launch("gated_delta_norm_param_grad_kernel");
}

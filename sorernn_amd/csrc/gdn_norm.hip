// Row-wise epilogue/prologue norms: L2 normalisation (q/k) and gated RMSNorm (GDN output).
//
// One wave per row (rows of D = 64 or 128 elements in the GDN path, any D here): each lane reads
// D/64 elements, the sum of squares is reduced across the wave, and the row is written once with
// fp32 math and a single rounding. Both kernels are HBM-bound elementwise passes.

#include "gdn_common.h"

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
  int mode;  // 0 = L2 norm, 1 = (gated) RMSNorm
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
          out *= (p.act == GDN_ACT_SILU) ? silu_f32(gv) : gv;
        }
      }
      store_from_f32(p.y, p.dt, base + e, out);
    }
  }
}

static int launch_norm(const NormParams& p, void* stream, const char* what) {
  if (p.rows == 0) return GDN_OK;
  int64_t blocks = (p.rows + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(gated_delta_norm_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  return gdn_internal_check_launch(what);
}

}  // namespace gdn

using namespace gdn;

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

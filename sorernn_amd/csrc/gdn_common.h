// Shared device helpers for the gfx950 Gated DeltaNet kernels: element types, conversions,
// wave-level reductions, the MFMA fragment types and the library's error channel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdn.h"

namespace gdn {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- element access by runtime dtype
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case GDN_DTYPE_BF16: return static_cast<float>(static_cast<const bf16*>(p)[i]);
    case GDN_DTYPE_F16: return static_cast<float>(static_cast<const f16*>(p)[i]);
    default: return static_cast<const float*>(p)[i];
  }
}

__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float x) {
  switch (dtype) {
    case GDN_DTYPE_BF16: static_cast<bf16*>(p)[i] = static_cast<bf16>(x); break;
    case GDN_DTYPE_F16: static_cast<f16*>(p)[i] = static_cast<f16>(x); break;
    default: static_cast<float*>(p)[i] = x; break;
  }
}

// Round an fp32 value to the storage dtype and back (the value a store followed by a load sees).
__device__ __forceinline__ float round_to(int dtype, float x) {
  switch (dtype) {
    case GDN_DTYPE_BF16: return static_cast<float>(static_cast<bf16>(x));
    case GDN_DTYPE_F16: return static_cast<float>(static_cast<f16>(x));
    default: return x;
  }
}

// Raw bits of element i (fp32 as is, 16-bit types zero-extended): a load with no conversion, so the
// wait for it can be deferred to the first use.
__device__ __forceinline__ uint32_t load_raw32(const void* p, int dtype, int64_t i) {
  if (dtype == GDN_DTYPE_F32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ float raw32_to_f32(uint32_t bits, int dtype) {
  switch (dtype) {
    case GDN_DTYPE_BF16: return __uint_as_float(bits << 16);
    case GDN_DTYPE_F16: return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits)));
    default: return __uint_as_float(bits);
  }
}

__device__ __forceinline__ int64_t load_index(const void* p, int is_i32, int64_t i) {
  return is_i32 ? static_cast<int64_t>(static_cast<const int32_t*>(p)[i]) : static_cast<const int64_t*>(p)[i];
}

// ---------------------------------------------------------------- scalar math
// softplus with torch's default threshold (beta=1, threshold=20): x for x > 20, else log1p(exp(x)).
__device__ __forceinline__ float softplus_f32(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float silu_f32(float x) { return x / (1.f + expf(-x)); }
// SiLU for kernels whose outputs are rounded to a 16-bit type: v_exp_f32 and v_rcp_f32 (about 2 ulp
// of fp32, far below the bf16/fp16 rounding) instead of the accurate expf and an IEEE divide.
// x -> -inf gives -0 (exp overflows to inf, rcp(inf) = 0); x -> +inf gives x.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// ---------------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_xor_sum(float x, int from_stride) {
  for (int s = from_stride; s < kWave; s <<= 1) x += __shfl_xor(x, s, kWave);
  return x;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP (no LDS): shifts of 1, 2, 4, 8 inside
// each row of 16 lanes, then row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
  return v + __int_as_float(s);
}

// Sum over aligned groups of N lanes (N = 8 or 16) with DPP: quad_perm [1,0,3,2] and [2,3,0,1]
// (0xb1, 0x4e), row_half_mirror (0x141, pairs the two quads of an 8-lane half) and row_mirror
// (0x140, pairs the two halves of a 16-lane row). Every lane of a group ends with the group sum.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 8 || N == 16, "group of 8 or 16 lanes");
  x = dpp_add<0xb1, 0xf>(x);
  x = dpp_add<0x4e, 0xf>(x);
  x = dpp_add<0x141, 0xf>(x);
  if (N == 16) x = dpp_add<0x140, 0xf>(x);
  return x;
}

__device__ __forceinline__ float wave_inclusive_sum(float x) {
  // DPP row_shr:n = 0x110 + n; row_bcast:15 = 0x142; row_bcast:31 = 0x143
  x = dpp_add<0x111, 0xf>(x);
  x = dpp_add<0x112, 0xf>(x);
  x = dpp_add<0x114, 0xf>(x);
  x = dpp_add<0x118, 0xf>(x);
  x = dpp_add<0x142, 0xa>(x);
  x = dpp_add<0x143, 0xc>(x);
  return x;
}

}  // namespace gdn

// Error channel shared by every entry point (defined in gdn_api.hip).
extern "C" void gdn_internal_set_error(const char* fmt, ...) __attribute__((visibility("hidden")));
extern "C" int gdn_internal_check_launch(const char* what) __attribute__((visibility("hidden")));

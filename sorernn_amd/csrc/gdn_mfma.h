// MFMA fragment helpers and the per-chunk building blocks shared by the two chunked-prefill
// kernels (the T-solve kernel and the state kernel) for gfx950.
//
// MFMA operand layouts used throughout (64 lanes, g = lane/16, i = lane%16):
//   v_mfma_f32_16x16x32_bf16: A lane holds row i, k = 8g..8g+7; B lane holds column i, same k;
//     the accumulator lane holds column i, rows 4g..4g+3.
//   v_mfma_f32_16x16x16_bf16 (1k): A row i, k = 4g..4g+3; B column i, same k; accumulator as
//     above, which is also this instruction's B-operand layout.
#pragma once

#include "gdn_common.h"

namespace gdn {

constexpr int kC = 64;       // chunk length (tokens)
constexpr int kCP = kC + 8;  // bf16 pitch of [*][64] operand tiles (144 B rows)
constexpr int kAoP = 52;     // fp32 pitch of the off-diagonal A rows 16..63 x cols 0..47
constexpr int kTfP = 36;     // fp32 pitch of the two 32x32 diagonal T blocks

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// x, with its value hidden from the optimiser: values derived from the result inside a loop are
// computed there instead of being hoisted out of the loop and kept in registers.
__device__ __forceinline__ int opaque_int(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ float4 ld4f(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mmah(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x8 ld8h(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }

// Transposed reads of a row-major bf16 LDS tile M (pitch in elements) with ds_read_b64_tr_b16.
// The instruction works inside groups of 16 lanes: each lane supplies 4 consecutive elements
// from its own address, and lane i receives element i % 4 of the lanes 4m + i / 4, m = 0..3.
// When lane 4m + q of group g reads row R_g + m at columns C_q..C_q+3, lane i of the group
// therefore receives M[R_g + m][C_{i/4} + i%4] for m = 0..3.
//
// ld4_tr: C_q = c0 + 4q, R_g = r0 + 4g: lane (g, i) gets M[r0 + 4g + m][c0 + i], m = 0..3 (the
// accumulator-layout fragment of a 16 x 16 tile at (r0, c0)).
__device__ __forceinline__ bf16x4 ld4_tr(const bf16* tile, int pitch, int r0, int c0, int lane) {
  const int g = lane >> 4, li = lane & 15;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (lds_bf16x4*)(tile + (r0 + 4 * g + (li >> 2)) * pitch + c0 + 4 * (li & 3)));
}
// ld8_tr_pair: C_q = c0 + 8q, rows r0 + 4g + m then r0 + 16 + 4g + m: lane (g, i) gets column
// c0 + 8(i/4) + i%4 at rows {r0 + 4g + m, r0 + 16 + 4g + m}, m = 0..3 -- the A operand of a
// 16x16x32 MFMA whose contraction index pairs two row tiles (16 rows apart) of M.
__device__ __forceinline__ bf16x8 ld8_tr_pair(const bf16* tile, int pitch, int r0, int c0, int lane) {
  const int g = lane >> 4, li = lane & 15;
  const bf16* p0 = tile + (r0 + 4 * g + (li >> 2)) * pitch + c0 + 8 * (li & 3);
  const bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0));
  const bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 16 * pitch));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ f16x8 ld8h_tr_pair(const f16* tile, int pitch, int r0, int c0, int lane) {
  return __builtin_bit_cast(f16x8, ld8_tr_pair(reinterpret_cast<const bf16*>(tile), pitch, r0, c0, lane));
}

// Contraction order of the chunk's token index used by the state kernel: a 16x16x32 MFMA whose
// B operand is a pair of accumulator tiles (rows 32u..32u+15 and 32u+16..32u+31) gives lane group
// g the tokens 32u + 4g + r and 32u + 16 + 4g + r, r = 0..3. T - I and P are stored with their
// columns in that order, so the matching A operand is one 16-byte row read: token
// j = 32u + 16h + 4g + r sits at column 32u + 8g + 4h + r.
__device__ __forceinline__ constexpr int tok_col(int j) {
  return (j & ~31) + 8 * ((j >> 2) & 3) + 4 * ((j >> 4) & 1) + (j & 3);
}

// Two fp32 accumulator fragments (4 elements each) as one bf16 / fp16 MFMA operand of 8
__device__ __forceinline__ bf16x8 pack8(f32x4 a, f32x4 b) {
  return bf16x8{static_cast<bf16>(a[0]), static_cast<bf16>(a[1]), static_cast<bf16>(a[2]), static_cast<bf16>(a[3]),
                static_cast<bf16>(b[0]), static_cast<bf16>(b[1]), static_cast<bf16>(b[2]), static_cast<bf16>(b[3])};
}
__device__ __forceinline__ f16x8 pack8h(f32x4 a, f32x4 b) {
  return f16x8{static_cast<f16>(a[0]), static_cast<f16>(a[1]), static_cast<f16>(a[2]), static_cast<f16>(a[3]),
               static_cast<f16>(b[0]), static_cast<f16>(b[1]), static_cast<f16>(b[2]), static_cast<f16>(b[3])};
}
// bf16 -> fp16, exact for magnitudes in [2^-14, 65504]
__device__ __forceinline__ f16x8 bf16_to_f16x8(bf16x8 x) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = static_cast<f16>(static_cast<float>(x[i]));
  return r;
}

// ---------------------------------------------------------------- raw buffer access
// A buffer resource covers [base, base + bytes); a load past the end returns zeros and a store
// past the end is dropped by the hardware range check. The loads are therefore unconditional
// instructions (no branch around them, no zero fill of the destination in between), which keeps
// the vector-memory counter waits at the points where the data is used.
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit dword format, no swizzle
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ bf16x8 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ void buf_store16(bf16x8 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)off, 0, 0);
}
// Raw bits of one gate element (fp32 as is, 16-bit types zero-extended), like load_raw32.
__device__ __forceinline__ uint32_t buf_load_raw32(__amdgpu_buffer_rsrc_t r, uint32_t off, int dtype) {
  if (dtype == GDN_DTYPE_F32) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ int dtype_bytes(int dtype) { return dtype == GDN_DTYPE_F32 ? 4 : 2; }

// Value of lane (quad base + q) broadcast to the 4 lanes of each quad (DPP quad_perm q,q,q,q).
__device__ __forceinline__ float quad_bcast(float x, int q) {
  const int v = __float_as_int(x);
  switch (q) {
    case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x00, 0xf, 0xf, false));
    case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x55, 0xf, 0xf, false));
    case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xaa, 0xf, 0xf, false));
    default: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xff, 0xf, 0xf, false));
  }
}

__device__ __forceinline__ bf16x4 to_bf16x4(float a, float b, float c, float d) {
  return bf16x4{static_cast<bf16>(a), static_cast<bf16>(b), static_cast<bf16>(c), static_cast<bf16>(d)};
}
__device__ __forceinline__ f16x4 to_f16x4(float a, float b, float c, float d) {
  return f16x4{static_cast<f16>(a), static_cast<f16>(b), static_cast<f16>(c), static_cast<f16>(d)};
}

// Per-token gate terms of one chunk: gam = in-chunk cumsum of g, egam = exp(gam), bet = beta,
// begam = beta exp(gam), dlast = exp(gam_last - gam). Padding rows carry g = 0 and beta = 0.
struct ChunkGates {
  float gam[kC], egam[kC], bet[kC], begam[kC], dlast[kC];
};

// One wave (lane = token) turns the raw gate bits of a chunk into its ChunkGates: optional
// in-kernel gate (g = -exp(A_log) softplus(a + dt_bias)) and sigmoid of beta, then a DPP scan.
__device__ __forceinline__ void chunk_gates_from_raw(ChunkGates& gs, uint32_t graw, uint32_t braw, int dg, int db,
                                                     int valid_rows, unsigned flags, float A_log, float dt_bias,
                                                     int lane) {
  float gval = raw32_to_f32(graw, dg), bval = raw32_to_f32(braw, db);
  if (lane < valid_rows) {
    // softplus and sigmoid from v_exp_f32 / v_log_f32 / v_rcp_f32 (this runs once per chunk on a
    // wave that shares its SIMD with a state wave). softplus(x) = ln(1 + e^x) for x <= 20 loses
    // only ~e^x absolutely where 1 + e^x rounds to 1, i.e. |error in g| <= exp(A_log) * 1e-7.
    constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;
    if (flags & GDN_FLAG_GATE_IN_KERNEL) {
      const float x = gval + dt_bias;
      const float sp = x > 20.f ? x : __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(x * kLog2e)) * kLn2;
      gval = -__builtin_amdgcn_exp2f(A_log * kLog2e) * sp;
    }
    if (flags & GDN_FLAG_BETA_SIGMOID) bval = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-bval * kLog2e));
  } else {
    gval = 0.f;
    bval = 0.f;
  }
  const float cs = wave_inclusive_sum(gval);
  const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cs), kWave - 1));
  const float e = __expf(cs);
  gs.gam[lane] = cs;
  gs.egam[lane] = e;
  gs.bet[lane] = bval;
  gs.begam[lane] = bval * e;
  gs.dlast[lane] = __expf(last - cs);
}

// F.normalize over a q/k row held by KCH consecutive lanes (8 bf16 each), rounded back to bf16.
// 1 / max(||x||, 1e-12) as v_rsq_f32 of max(||x||^2, 1e-24): about 1 ulp of fp32 from the IEEE
// sqrt and divide, far below the bf16 rounding that follows, and a few instructions instead of the
// IEEE sequences (this runs on the helper waves once per 16-byte chunk of every q/k row).
template <int KCH>
__device__ __forceinline__ bf16x8 l2norm_row_chunk(bf16x8 x) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += (float)x[i] * (float)x[i];
  ss = group_sum<KCH>(ss);
  const float inv = __builtin_amdgcn_rsqf(fmaxf(ss, 1e-24f));
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<bf16>((float)x[i] * inv);
  return x;
}

}  // namespace gdn

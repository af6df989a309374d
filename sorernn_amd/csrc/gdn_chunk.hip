// Fused chunked gated delta rule forward (prefill) for gfx950: bf16 MFMA, 64-token chunks, the fp32
// state held in MFMA accumulators across the whole sequence.
//
// Work split: one workgroup (4 waves) per (sequence, value head, 32-column slice of V). The state
// columns evolve independently, so the slice's state S_b [K x 32] never leaves the workgroup; the
// K-side of a chunk (k.k and k.q Gram tiles, the triangular solve) is recomputed by each of the
// V/32 slices. Workgroups of one (sequence, head) are placed on the same XCD so the q/k tiles they
// all read come from one L2.
//
// Per chunk of c <= 64 tokens with gam = in-chunk cumsum of g (sore/model/gdn_ref.py:17-21 in
// chunk form, the algebra restated in oracle/gdn_oracle.py::_chunk_segment):
//   A_tj  = beta_t exp(gam_t - gam_j) k_t.k_j   (j < t)          T = (I + A)^-1
//   X     = diag(beta) V - diag(beta exp(gam)) K S              Delta = T X = X + (T - I) X
//   O     = scale (diag(exp(gam)) Q S + P Delta),  P_tj = exp(gam_t - gam_j) q_t.k_j  (j <= t)
//   S'    = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta
// Precision: q/k/v are bf16 already, so the Gram tiles are exact products with fp32 accumulation.
// S, X and Delta enter MFMA as single bf16; the state update's right operand is split into bf16
// hi + lo (two MFMAs), which keeps the fp32 final state within 1e-3 relative L2 over 64 chunks.
// T is built in fp32: the four 16x16 diagonal blocks by forward substitution, then two merge levels
// (16 -> 32 -> 64) with fp32 MFMA.
//
// LDS operand layouts (bf16 rows padded by 8 elements):
//   Kc, Qc [token][key]  natural tiles: A/B operands with the key dim contiguous; K^T for the state
//                        update is read with ds_read_b64_tr_b16 (token-contiguous fragments).
//   Sb [v][key], Xb/Db/DtH/DtL [v][token], Tb/Pb [t][j]: written from accumulators with 8-byte stores.

#include "gdn_common.h"

namespace gdn {

struct ChunkParams {
  const void *q, *k, *v, *g, *beta;
  const float* h0;
  void* o;
  float* ht;
  const void* cu;
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
};

constexpr int kC = 64;       // chunk length
constexpr int kVB = 32;      // value columns per workgroup
constexpr int kNT = 256;     // threads per workgroup (4 waves)
constexpr int kCP = kC + 8;  // bf16 pitch of [*][64] operand tiles (144 B rows)
constexpr int kFP = kC + 4;  // fp32 pitch of 64x64 matrices (272 B rows)
constexpr int kVP = kVB + 8;  // bf16 pitch of the V slice (80 B rows)

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Transposed A/B fragment from a row-major bf16 LDS tile M (pitch in elements): lane (g = lane/16,
// i = lane%16) receives M[j0 + 8g + m][c0 + i] for m = 0..7, i.e. the fragment of M^T with rows
// c0.. and the contraction index j0.. contiguous. Each ds_read_b64_tr_b16 covers 4 rows: inside a
// group of 16 lanes, lane 4m+q reads row m at columns c0+4q..+3 and the instruction hands lane i
// the element i%4 of lanes 4m + i/4, m = 0..3.
__device__ __forceinline__ bf16x8 ld8_tr(const bf16* tile, int pitch, int j0, int c0, int lane) {
  const int g = lane >> 4, li = lane & 15;
  const bf16* p0 = tile + (j0 + 8 * g + (li >> 2)) * pitch + c0 + 4 * (li & 3);
  const bf16* p1 = p0 + 4 * pitch;
  const bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0));
  const bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p1));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ bf16x4 to_bf16x4(float a, float b, float c, float d) {
  return bf16x4{static_cast<bf16>(a), static_cast<bf16>(b), static_cast<bf16>(c), static_cast<bf16>(d)};
}

template <int KD, int VD>
__global__ __launch_bounds__(kNT, 1) void gated_delta_chunk_kernel(ChunkParams p) {
  constexpr int NVB = VD / kVB;
  constexpr int KP = KD + 8;       // bf16 pitch of the q/k tiles
  constexpr int KS = KD / 32;      // MFMA k-steps over the key dim
  constexpr int SMT = KD / 64;     // 16-row state tiles per wave
  constexpr int KCH = KD / 8;      // 16-byte chunks per q/k row

  __shared__ __align__(16) bf16 Kc[kC * KP];
  __shared__ __align__(16) bf16 Qc[kC * KP];
  __shared__ __align__(16) bf16 Vc[kC * kVP];
  __shared__ __align__(16) bf16 Sb[kVB * KP];
  __shared__ __align__(16) float Af[kC * kFP];
  __shared__ __align__(16) float Tf[kC * kFP];
  __shared__ __align__(16) bf16 Tb[kC * kCP];
  __shared__ __align__(16) bf16 Pb[kC * kCP];
  __shared__ __align__(16) bf16 Xb[kVB * kCP];
  __shared__ __align__(16) bf16 Db[kVB * kCP];
  __shared__ __align__(16) bf16 DtH[kVB * kCP];
  __shared__ __align__(16) bf16 DtL[kVB * kCP];
  __shared__ float gam[kC], egam[kC], bet[kC], begam[kC], dlast[kC];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6, g4 = lane >> 4, li = lane & 15;

  // workgroup -> (sequence n, value head hv, slice vb); the NVB slices of a chain share an XCD
  const int64_t chains = p.N * p.HV;
  int64_t id = blockIdx.x;
  if (chains % 8 == 0) {
    const int64_t per = chains * NVB / 8;
    id = (id % 8) * per + id / 8;
  }
  const int vb = (int)(id % NVB);
  const int64_t chain = id / NVB;
  const int hv = (int)(chain % p.HV);
  const int64_t n = chain / p.HV;
  const int h = hv / (int)(p.HV / p.H);
  int64_t bos, eos;
  if (p.cu) {
    bos = load_index(p.cu, p.cu_i32, n);
    eos = load_index(p.cu, p.cu_i32, n + 1);
  } else {
    bos = n * p.T;
    eos = bos + p.T;
  }
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const bf16* __restrict__ qg = static_cast<const bf16*>(p.q);
  const bf16* __restrict__ kg = static_cast<const bf16*>(p.k);
  const bf16* __restrict__ vg = static_cast<const bf16*>(p.v);
  bf16* __restrict__ og = static_cast<bf16*>(p.o);

  // T - I and P are strictly/causally lower: their upper blocks stay zero for the whole run
  for (int e = t; e < kC * kCP / 8; e += kNT) {
    reinterpret_cast<bf16x8*>(Tb)[e] = bf16x8{};
    reinterpret_cast<bf16x8*>(Pb)[e] = bf16x8{};
  }

  // state slice: wave w owns key rows [16*SMT*w, 16*SMT*(w+1)) x 32 columns as 2*SMT accumulators
  f32x4 sacc[SMT][2];
  const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVB;
#pragma unroll
  for (int mt = 0; mt < SMT; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int kd0 = 16 * (w * SMT + mt) + 4 * g4, vv = 16 * nt + li;
#pragma unroll
      for (int i = 0; i < 4; ++i) sacc[mt][nt][i] = p.h0 ? p.h0[sbase + (int64_t)(kd0 + i) * VD + vv] : 0.f;
      *reinterpret_cast<bf16x4*>(Sb + vv * KP + kd0) =
          to_bf16x4(sacc[mt][nt][0], sacc[mt][nt][1], sacc[mt][nt][2], sacc[mt][nt][3]);
    }
  }

  for (int64_t c0 = bos; c0 < eos; c0 += kC) {
    const int len = (int)((eos - c0) < kC ? (eos - c0) : kC);
    // ---------------------------------------------------------------- stage the chunk
    for (int e = t; e < kC * KCH; e += kNT) {
      const int row = e / KCH, c8 = e % KCH;
      bf16x8 kv{}, qv{};
      if (row < len) {
        const int64_t base = ((c0 + row) * p.H + h) * KD + c8 * 8;
        kv = *reinterpret_cast<const bf16x8*>(kg + base);
        qv = *reinterpret_cast<const bf16x8*>(qg + base);
      }
      if (l2) {  // F.normalize over the row: KCH consecutive lanes hold one row
        float sk = 0.f, sq = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          sk += (float)kv[i] * (float)kv[i];
          sq += (float)qv[i] * (float)qv[i];
        }
#pragma unroll
        for (int off = 1; off < KCH; off <<= 1) {
          sk += __shfl_xor(sk, off, kWave);
          sq += __shfl_xor(sq, off, kWave);
        }
        const float ik = 1.f / fmaxf(sqrtf(sk), 1e-12f), iq = 1.f / fmaxf(sqrtf(sq), 1e-12f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kv[i] = static_cast<bf16>((float)kv[i] * ik);
          qv[i] = static_cast<bf16>((float)qv[i] * iq);
        }
      }
      *reinterpret_cast<bf16x8*>(Kc + row * KP + c8 * 8) = kv;
      *reinterpret_cast<bf16x8*>(Qc + row * KP + c8 * 8) = qv;
    }
    {
      const int row = t >> 2, c8 = t & 3;  // 64 rows x 4 chunks of 8 = 256 threads
      bf16x8 vv{};
      if (row < len) vv = *reinterpret_cast<const bf16x8*>(vg + ((c0 + row) * p.HV + hv) * VD + vb * kVB + c8 * 8);
      *reinterpret_cast<bf16x8*>(Vc + row * kVP + c8 * 8) = vv;
    }
    if (w == 0) {  // gates and the in-chunk cumsum of g (padding rows: g = 0, beta = 0)
      float gv = 0.f, bv = 0.f;
      if (lane < len) {
        const int64_t gi = (c0 + lane) * p.HV + hv;
        gv = load_as_f32(p.g, p.dg, gi);
        if (p.flags & GDN_FLAG_GATE_IN_KERNEL) gv = -expf(p.A_log[hv]) * softplus_f32(gv + p.dt_bias[hv]);
        bv = load_as_f32(p.beta, p.db, gi);
        if (p.flags & GDN_FLAG_BETA_SIGMOID) bv = sigmoid_f32(bv);
      }
      float cs = gv;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const float y = __shfl_up(cs, off, kWave);
        if (lane >= off) cs += y;
      }
      const float last = __shfl(cs, kWave - 1, kWave);
      const float e = expf(cs);
      gam[lane] = cs;
      egam[lane] = e;
      bet[lane] = bv;
      begam[lane] = bv * e;
      dlast[lane] = expf(last - cs);
    }
    __syncthreads();

    // ---------------------------------------------------------------- Gram tiles, K S and Q S
    // 20 jobs: upper tiles (rb <= cb) of K K^T (-> A) and of K Q^T (-> P); element (r, c) of tile
    // (rb, cb) is row j = r, column t = c, so the accumulator writes 4 consecutive j of row t.
#pragma unroll
    for (int jj = 0; jj < 5; ++jj) {
      const int job = w + 4 * jj;
      const bool isq = job >= 10;
      const int tj = isq ? job - 10 : job;
      const int rb = tj < 4 ? 0 : tj < 7 ? 1 : tj < 9 ? 2 : 3;
      const int cb = tj < 4 ? tj : tj < 7 ? tj - 3 : tj < 9 ? tj - 5 : 3;
      const bf16* bsrc = isq ? Qc : Kc;
      f32x4 acc{};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = mma(ld8(Kc + (16 * rb + li) * KP + 32 * s + 8 * g4), ld8(bsrc + (16 * cb + li) * KP + 32 * s + 8 * g4), acc);
      const int tt = 16 * cb + li, j0 = 16 * rb + 4 * g4;
      const float gt = gam[tt];
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = j0 + i;
        const bool keep = isq ? (j <= tt) : (j < tt);
        val[i] = keep ? expf(gt - gam[j]) * acc[i] : 0.f;
      }
      if (isq) {
        *reinterpret_cast<bf16x4*>(Pb + tt * kCP + j0) = to_bf16x4(val[0], val[1], val[2], val[3]);
      } else {
        const float bt = bet[tt];
        *reinterpret_cast<float4*>(Af + tt * kFP + j0) = make_float4(bt * val[0], bt * val[1], bt * val[2], bt * val[3]);
      }
    }
    f32x4 yacc[2] = {}, zacc[2] = {};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bf16x8 ak = ld8(Kc + (16 * w + li) * KP + 32 * s + 8 * g4);
      const bf16x8 aq = ld8(Qc + (16 * w + li) * KP + 32 * s + 8 * g4);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const bf16x8 b = ld8(Sb + (16 * nt + li) * KP + 32 * s + 8 * g4);
        yacc[nt] = mma(ak, b, yacc[nt]);
        zacc[nt] = mma(aq, b, zacc[nt]);
      }
    }
    // X = beta V - beta e^gam (K S), rows j = 16w + 4g + i; kept in fp32 for the identity part of T
    f32x4 xacc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int vv = 16 * nt + li;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * w + 4 * g4 + i;
        xacc[nt][i] = bet[j] * (float)Vc[j * kVP + vv] - begam[j] * yacc[nt][i];
      }
      *reinterpret_cast<bf16x4*>(Xb + vv * kCP + 16 * w + 4 * g4) = to_bf16x4(xacc[nt][0], xacc[nt][1], xacc[nt][2], xacc[nt][3]);
    }
    __syncthreads();

    // ---------------------------------------------------------------- T = (I + A)^-1
    if (w == 0) {  // diagonal 16x16 blocks: lane (b, c) solves column c of block b
      const int b = g4, c = li;
      const float* ab = Af + 16 * b * kFP + 16 * b;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = (r == c) ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const float xm = x[m];
#pragma unroll
        for (int r = m + 1; r < 16; ++r) x[r] -= ab[r * kFP + m] * xm;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        Tf[(16 * b + r) * kFP + 16 * b + c] = x[r];
        Tb[(16 * b + r) * kCP + 16 * b + c] = static_cast<bf16>(r == c ? 0.f : x[r]);
      }
    }
    __syncthreads();
    if (w < 2) {  // 16 -> 32: W = A_{2q+1,2q} T_{2q,2q} into the unused upper block (2q, 2q+1)
      const int R = 16 * (2 * w + 1), Cc = 16 * (2 * w);
      f32x4 acc{};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc = mma_f32(Af[(R + li) * kFP + Cc + 4 * s + g4], Tf[(Cc + 4 * s + g4) * kFP + Cc + li], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) Tf[(Cc + 4 * g4 + i) * kFP + R + li] = acc[i];
    }
    __syncthreads();
    if (w < 2) {  // T_{2q+1,2q} = -T_{2q+1,2q+1} W
      const int R = 16 * (2 * w + 1), Cc = 16 * (2 * w);
      f32x4 acc{};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc = mma_f32(Tf[(R + li) * kFP + R + 4 * s + g4], Tf[(Cc + 4 * s + g4) * kFP + R + li], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        Tf[(R + 4 * g4 + i) * kFP + Cc + li] = -acc[i];
        Tb[(R + 4 * g4 + i) * kCP + Cc + li] = static_cast<bf16>(-acc[i]);
      }
    }
    __syncthreads();
    {  // 32 -> 64: W' = A[32:64][0:32] T[0:32][0:32] into the unused upper block [0:32][32:64]
      const int rt = w >> 1, ct = w & 1;
      f32x4 acc{};
#pragma unroll
      for (int s = 4 * ct; s < 8; ++s)
        acc = mma_f32(Af[(32 + 16 * rt + li) * kFP + 4 * s + g4], Tf[(4 * s + g4) * kFP + 16 * ct + li], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) Tf[(16 * rt + 4 * g4 + i) * kFP + 32 + 16 * ct + li] = acc[i];
    }
    __syncthreads();
    {  // T[32:64][0:32] = -T[32:64][32:64] W'
      const int rt = w >> 1, ct = w & 1;
      f32x4 acc{};
      for (int s = 0; s < 4 * rt + 4; ++s)
        acc = mma_f32(Tf[(32 + 16 * rt + li) * kFP + 32 + 4 * s + g4], Tf[(4 * s + g4) * kFP + 32 + 16 * ct + li], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) Tb[(32 + 16 * rt + 4 * g4 + i) * kCP + 16 * ct + li] = static_cast<bf16>(-acc[i]);
    }
    __syncthreads();

    // ---------------------------------------------------------------- Delta = X + (T - I) X
    f32x4 dacc[2] = {xacc[0], xacc[1]};
    const int ksteps = (w >= 2) ? 2 : 1;  // (T - I) and P vanish for j > t
    for (int s = 0; s < ksteps; ++s) {
      const bf16x8 a = ld8(Tb + (16 * w + li) * kCP + 32 * s + 8 * g4);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) dacc[nt] = mma(a, ld8(Xb + (16 * nt + li) * kCP + 32 * s + 8 * g4), dacc[nt]);
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int vv = 16 * nt + li, tb = 16 * w + 4 * g4;
      *reinterpret_cast<bf16x4*>(Db + vv * kCP + tb) = to_bf16x4(dacc[nt][0], dacc[nt][1], dacc[nt][2], dacc[nt][3]);
      float hi[4], lo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d = dlast[tb + i] * dacc[nt][i];
        hi[i] = (float)static_cast<bf16>(d);
        lo[i] = d - hi[i];
      }
      *reinterpret_cast<bf16x4*>(DtH + vv * kCP + tb) = to_bf16x4(hi[0], hi[1], hi[2], hi[3]);
      *reinterpret_cast<bf16x4*>(DtL + vv * kCP + tb) = to_bf16x4(lo[0], lo[1], lo[2], lo[3]);
    }
    __syncthreads();

    // ---------------------------------------------------------------- O = scale (e^gam Q S + P Delta)
    {
      f32x4 oacc[2] = {};
      for (int s = 0; s < ksteps; ++s) {
        const bf16x8 a = ld8(Pb + (16 * w + li) * kCP + 32 * s + 8 * g4);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) oacc[nt] = mma(a, ld8(Db + (16 * nt + li) * kCP + 32 * s + 8 * g4), oacc[nt]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tt = 16 * w + 4 * g4 + i;
        if (tt < len) {
          bf16* orow = og + ((c0 + tt) * p.HV + hv) * VD + vb * kVB + li;
          const float eg = egam[tt];
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) orow[16 * nt] = static_cast<bf16>(p.scale * (eg * zacc[nt][i] + oacc[nt][i]));
        }
      }
    }
    // ---------------------------------------------------------------- S' = e^{gam_c} S + K^T Delta~
    {
      const float ec = expf(gam[kC - 1]);
#pragma unroll
      for (int mt = 0; mt < SMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) sacc[mt][nt] *= ec;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int mt = 0; mt < SMT; ++mt) {
          const bf16x8 a = ld8_tr(Kc, KP, 32 * s, 16 * (w * SMT + mt), lane);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            const int off = (16 * nt + li) * kCP + 32 * s + 8 * g4;
            sacc[mt][nt] = mma(a, ld8(DtH + off), sacc[mt][nt]);
            sacc[mt][nt] = mma(a, ld8(DtL + off), sacc[mt][nt]);
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < SMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          *reinterpret_cast<bf16x4*>(Sb + (16 * nt + li) * KP + 16 * (w * SMT + mt) + 4 * g4) =
              to_bf16x4(sacc[mt][nt][0], sacc[mt][nt][1], sacc[mt][nt][2], sacc[mt][nt][3]);
    }
    __syncthreads();
  }

  if (p.ht) {
#pragma unroll
    for (int mt = 0; mt < SMT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int kd0 = 16 * (w * SMT + mt) + 4 * g4, vv = 16 * nt + li;
#pragma unroll
        for (int i = 0; i < 4; ++i) p.ht[sbase + (int64_t)(kd0 + i) * VD + vv] = sacc[mt][nt][i];
      }
  }
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                             const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                             int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                             int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                             const float* A_log, const float* dt_bias, void* stream) {
  if (!q || !k || !v || !g || !beta || !o) {
    gdn_internal_set_error("gdn_chunk_fwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || H <= 0 || HV <= 0 || HV % H || N <= 0) {
    gdn_internal_set_error("gdn_chunk_fwd: bad sizes B=%lld T=%lld H=%lld HV=%lld N=%lld", (long long)B, (long long)T,
                           (long long)H, (long long)HV, (long long)N);
    return GDN_ERR_INVALID;
  }
  if (cu_seqlens ? B != 1 : N != B) {
    gdn_internal_set_error("gdn_chunk_fwd: cu_seqlens requires B == 1 (and N == B without it)");
    return GDN_ERR_INVALID;
  }
  if ((flags & GDN_FLAG_GATE_IN_KERNEL) && (!A_log || !dt_bias)) {
    gdn_internal_set_error("gdn_chunk_fwd: gate in kernel needs A_log and dt_bias");
    return GDN_ERR_INVALID;
  }
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) {
    gdn_internal_set_error("gdn_chunk_fwd: head dims K=%lld V=%lld unsupported (each must be 64 or 128)", (long long)K,
                           (long long)V);
    return GDN_ERR_UNSUPPORTED;
  }
  if (qkv_dtype != GDN_DTYPE_BF16) {
    gdn_internal_set_error("gdn_chunk_fwd: q/k/v dtype %d unsupported by the chunk kernel (bf16 only)", qkv_dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  ChunkParams p{q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, (flags & GDN_FLAG_CU_INT32) ? 1 : 0,
                T, H, HV, N, g_dtype, beta_dtype, scale, flags, A_log, dt_bias};
  const int64_t blocks = N * HV * (V / kVB);
  if (blocks > 0x7fffffff) {
    gdn_internal_set_error("gdn_chunk_fwd: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)blocks), block(kNT);
  if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 128>), grid, block, 0, s, p);
  else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 64>), grid, block, 0, s, p);
  else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 64>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 128>), grid, block, 0, s, p);
  return gdn_internal_check_launch("gated_delta_chunk_kernel");
}

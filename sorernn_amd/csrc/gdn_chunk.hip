// Fused chunked gated delta rule forward (prefill) for gfx950: bf16 MFMA, 64-token chunks, the fp32
// state held in MFMA accumulators across the whole sequence.
//
// Work split: one workgroup (8 waves, two per SIMD) per (sequence, value head, 32-column slice of V).
// The state columns evolve independently, so the slice's state S_b [K x 32] never leaves the
// workgroup; the K-side of a chunk (Gram tiles and the triangular solve) is recomputed by each of the
// V/32 slices. The slices of one (sequence, head) are placed on the same XCD, so the q/k tiles they
// all read come from one L2.
//
// Per chunk of c <= 64 tokens with gam = in-chunk cumsum of g (sore/model/gdn_ref.py:17-21 in
// chunk form; the algebra is restated in oracle/gdn_oracle.py::_chunk_segment):
//   A_tj  = beta_t exp(gam_t - gam_j) k_t.k_j   (j < t)          T = (I + A)^-1
//   X     = diag(beta) V - diag(beta exp(gam)) K S              Delta = T X = X + (T - I) X
//   O     = scale (diag(exp(gam)) Q S + P Delta),  P_tj = exp(gam_t - gam_j) q_t.k_j  (j <= t)
//   S'    = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta
//
// Two-stage software pipeline: iteration i runs the state-dependent work of chunk i (S-side) and
// the state-independent work of chunk i+1 (K-side: A, the diagonal 16x16 inverses, the 16->32->64
// merges of T), so the solve's latency overlaps the state chain. Phases (one barrier each):
//   A: S: Y = K S, Z = Q S, X, P.        K: Gram k.k tiles -> A; diagonal inverses of T.
//   B: S: Delta = X + (T - I) X.         K: 16 -> 32 merges of T.
//   C: S: O, S' = e^{gam_c} S + K^T Delta~.   K: 32 -> 64 merge of T.
//   stage: write the prefetched tiles of the chunk after next (global loads issued in phase A).
//
// Precision: q/k/v are bf16, so Gram tiles are exact products with fp32 accumulation. S, X and
// Delta enter MFMA as single bf16; the state update's right operand is split into bf16 hi + lo (two
// MFMAs), which keeps the fp32 final state within 1e-3 relative L2 over 64 chunks. T is built in
// fp32: diagonal blocks by forward substitution, merges with three-term bf16 products
// (hi*hi + hi*lo + lo*hi, about 2^-16 relative), and rounded to bf16 once as an MFMA operand.
//
// LDS operand layouts (bf16 rows padded by 8 elements):
//   Kc, Qc [token][key]  natural tiles (two chunk buffers): A/B operands with the key dim contiguous;
//                        K^T for the state update is read with ds_read_b64_tr_b16.
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

constexpr int kC = 64;        // chunk length
constexpr int kVB = 32;       // value columns per workgroup
constexpr int kNT = 512;      // threads per workgroup (8 waves)
constexpr int kCP = kC + 8;   // bf16 pitch of [*][64] operand tiles (144 B rows)
constexpr int kVP = kVB + 8;  // bf16 pitch of the V slice (80 B rows)
constexpr int kAdP = 20;      // fp32 pitch of the diagonal A blocks
constexpr int kAoP = 52;      // fp32 pitch of the off-diagonal A rows 16..63 x cols 0..47
constexpr int kTfP = 36;      // fp32 pitch of the two 32x32 T blocks

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}

// Transposed fragment from a row-major bf16 LDS tile M (pitch in elements): lane (g = lane/16,
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

// fp32 x4 -> bf16 hi and lo parts (x ~= hi + lo to about 2^-16 relative)
__device__ __forceinline__ void split4(float a, float b, float c, float d, bf16x4& hi, bf16x4& lo) {
  hi = to_bf16x4(a, b, c, d);
  lo = to_bf16x4(a - (float)hi[0], b - (float)hi[1], c - (float)hi[2], d - (float)hi[3]);
}

// Three-term bf16 product step for a 16x16x16 fp32 tile: acc += A(4 k) * B(4 k).
__device__ __forceinline__ f32x4 mma16x3(const float (&a)[4], const float (&b)[4], f32x4 acc) {
  bf16x4 ah, al, bh, bl;
  split4(a[0], a[1], a[2], a[3], ah, al);
  split4(b[0], b[1], b[2], b[3], bh, bl);
  acc = mma16(ah, bh, acc);
  acc = mma16(ah, bl, acc);
  acc = mma16(al, bh, acc);
  return acc;
}

struct ChunkSmem {
  float gam[2][kC], egam[2][kC], bet[2][kC], begam[2][kC], dlast[2][kC];
};

template <int KD, int VD>
__global__ __launch_bounds__(kNT, 1) void gated_delta_chunk_kernel(ChunkParams p) {
  constexpr int NVB = VD / kVB;
  constexpr int KP = KD + 8;       // bf16 pitch of the q/k tiles
  constexpr int KS = KD / 32;      // MFMA k-steps over the key dim
  constexpr int KCH = KD / 8;      // 16-byte chunks per q/k row
  constexpr int QKPT = kC * KCH / kNT;  // q/k 16-byte chunks per thread per matrix
  // State tiles (16 x 16; KD/8 of them) owned per wave: waves 0-1 hold KD/32 each, waves 4-7 KD/64
  // each, waves 2-3 none (they run the 32 -> 64 merge of T in phase C instead).
  constexpr int SMAX = KD / 32;

  __shared__ __align__(16) bf16 Kc[2][kC * KP];
  __shared__ __align__(16) bf16 Qc[2][kC * KP];
  __shared__ __align__(16) bf16 Vc[kC * kVP];
  __shared__ __align__(16) bf16 Sb[kVB * KP];
  __shared__ __align__(16) float Ad[4][16 * kAdP];       // diagonal A blocks, row-major: Ad[b][r][m] = A[16b+r][16b+m]
  __shared__ __align__(16) float Ao[48 * kAoP];          // A rows 16..63 x cols 0..47 (off-diagonal lower blocks)
  __shared__ __align__(16) float Tf[2][32 * kTfP];       // T[0:32][0:32] and T[32:64][32:64] in fp32
  __shared__ __align__(16) bf16 Tb[2][kC * kCP];         // T - I in bf16, A operand [t][j], per chunk parity
  __shared__ __align__(16) bf16 Pb[kC * kCP];
  __shared__ __align__(16) bf16 Xb[kVB * kCP];
  __shared__ __align__(16) bf16 Db[kVB * kCP];
  __shared__ __align__(16) bf16 DtH[kVB * kCP];
  __shared__ __align__(16) bf16 DtL[kVB * kCP];
  __shared__ ChunkSmem gv;

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
  const int nc = (int)((eos - bos + kC - 1) / kC);
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const bf16* __restrict__ qg = static_cast<const bf16*>(p.q);
  const bf16* __restrict__ kg = static_cast<const bf16*>(p.k);
  const bf16* __restrict__ vg = static_cast<const bf16*>(p.v);
  bf16* __restrict__ og = static_cast<bf16*>(p.o);

  // ------------------------------------------------------------------ prefetch registers
  bf16x8 pk[QKPT], pq[QKPT], pv{};
  uint32_t pgraw = 0, pbraw = 0;  // gate bits as loaded (converted at the stage step)
  // K/Q/gates of chunk c (into registers)
  auto fetch_kq = [&](int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const int len = (int)((eos - c0) < kC ? (eos - c0) : kC);
#pragma unroll
    for (int u = 0; u < QKPT; ++u) {
      const int e = t + u * kNT, row = e / KCH, c8 = e % KCH;
      pk[u] = bf16x8{};
      pq[u] = bf16x8{};
      if (c < nc && row < len) {
        const int64_t base = ((c0 + row) * p.H + h) * KD + c8 * 8;
        pk[u] = *reinterpret_cast<const bf16x8*>(kg + base);
        pq[u] = *reinterpret_cast<const bf16x8*>(qg + base);
      }
    }
    pgraw = 0;
    pbraw = 0;
    if (w == 0 && c < nc && lane < len) {
      const int64_t gi = (c0 + lane) * p.HV + hv;
      pgraw = load_raw32(p.g, p.dg, gi);
      pbraw = load_raw32(p.beta, p.db, gi);
    }
  };
  auto fetch_v = [&](int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const int len = (int)((eos - c0) < kC ? (eos - c0) : kC);
    pv = bf16x8{};
    if (t < kC * 4 && c < nc) {
      const int row = t >> 2, c8 = t & 3;
      if (row < len) pv = *reinterpret_cast<const bf16x8*>(vg + ((c0 + row) * p.HV + hv) * VD + vb * kVB + c8 * 8);
    }
  };
  // registers -> LDS buffer `buf` (K/Q/gates) and the V slice
  auto stage_kq = [&](int buf, int valid_rows) {
#pragma unroll
    for (int u = 0; u < QKPT; ++u) {
      const int e = t + u * kNT, row = e / KCH, c8 = e % KCH;
      bf16x8 kv = pk[u], qv = pq[u];
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
      *reinterpret_cast<bf16x8*>(&Kc[buf][row * KP + c8 * 8]) = kv;
      *reinterpret_cast<bf16x8*>(&Qc[buf][row * KP + c8 * 8]) = qv;
    }
    if (w == 0) {  // gates and the in-chunk cumsum of g (padding rows: g = 0, beta = 0)
      float gval = raw32_to_f32(pgraw, p.dg), bval = raw32_to_f32(pbraw, p.db);
      if (lane < valid_rows) {
        if (p.flags & GDN_FLAG_GATE_IN_KERNEL) gval = -__expf(p.A_log[hv]) * softplus_f32(gval + p.dt_bias[hv]);
        if (p.flags & GDN_FLAG_BETA_SIGMOID) bval = sigmoid_f32(bval);
      }
      const float cs = wave_inclusive_sum(gval);
      const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cs), kWave - 1));
      const float e = __expf(cs);
      gv.gam[buf][lane] = cs;
      gv.egam[buf][lane] = e;
      gv.bet[buf][lane] = bval;
      gv.begam[buf][lane] = bval * e;
      gv.dlast[buf][lane] = __expf(last - cs);
    }
  };
  auto stage_v = [&]() {
    if (t < kC * 4) *reinterpret_cast<bf16x8*>(Vc + (t >> 2) * kVP + (t & 3) * 8) = pv;
  };

  // T - I and P are strictly/causally lower: their upper blocks stay zero for the whole run
  for (int e = t; e < kC * kCP / 8; e += kNT) {
    reinterpret_cast<bf16x8*>(Tb[0])[e] = bf16x8{};
    reinterpret_cast<bf16x8*>(Tb[1])[e] = bf16x8{};
    reinterpret_cast<bf16x8*>(Pb)[e] = bf16x8{};
  }

  // state slice: 16x16 tiles ti = s_first + u (u < s_count), row tile ti/2, column tile ti%2
  const int s_count = (w < 2) ? KD / 32 : (w >= 4 ? KD / 64 : 0);
  const int s_first = (w < 2) ? w * (KD / 32) : 2 * (KD / 32) + (w - 4) * (KD / 64);
  f32x4 sacc[SMAX];
  const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVB;
#pragma unroll
  for (int u = 0; u < SMAX; ++u) {
    if (u >= s_count) break;
    const int ti = s_first + u, kd0 = 16 * (ti >> 1) + 4 * g4, vv = 16 * (ti & 1) + li;
#pragma unroll
    for (int i = 0; i < 4; ++i) sacc[u][i] = p.h0 ? p.h0[sbase + (int64_t)(kd0 + i) * VD + vv] : 0.f;
    *reinterpret_cast<bf16x4*>(Sb + vv * KP + kd0) = to_bf16x4(sacc[u][0], sacc[u][1], sacc[u][2], sacc[u][3]);
  }

  fetch_kq(0);
  stage_kq(0, nc > 0 ? (int)((eos - bos) < kC ? (eos - bos) : kC) : 0);
  __syncthreads();

  f32x4 xacc[2], zacc[2];
  for (int i = -1; i < nc; ++i) {
    const bool s_on = i >= 0, k_on = i + 1 < nc;
    const int b0 = (i + 2) & 1, b1 = (i + 1) & 1;  // buffer of chunk i and of chunk i+1
    const int64_t c0 = bos + (int64_t)i * kC;
    const int len = s_on ? (int)((eos - c0) < kC ? (eos - c0) : kC) : 0;
    // prefetch: K/Q/gates of chunk i+2, V of chunk i+1 (held in registers until the stage step)
    fetch_kq(i + 2);
    fetch_v(i + 1);

    // ================================================================ phase A
    if (w < 4) {
      f32x4 yacc[2] = {};
      if (s_on) {  // Y = K S for row tile w (MFMAs issued first; the solve below overlaps them)
        const bf16* kb = Kc[b0];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 a = ld8(kb + (16 * w + li) * KP + 32 * s + 8 * g4);
          const bf16x8 s0 = ld8(Sb + li * KP + 32 * s + 8 * g4);
          const bf16x8 s1 = ld8(Sb + (16 + li) * KP + 32 * s + 8 * g4);
          yacc[0] = mma(a, s0, yacc[0]);
          yacc[1] = mma(a, s1, yacc[1]);
        }
      }
      if (k_on) {  // diagonal Gram tile (w, w) of chunk i+1 -> A block -> (I + A_ww)^-1
        const bf16* kb = Kc[b1];
        f32x4 acc{};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 f = ld8(kb + (16 * w + li) * KP + 32 * s + 8 * g4);
          acc = mma(f, f, acc);
        }
        // k.k is symmetric: acc[i] = k_t.k_j with t = 16w + li, j = 16w + 4g + i; A[t][j] for j < t
        const float gt = gv.gam[b1][16 * w + li], bt = gv.bet[b1][16 * w + li];
        float av[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int jl = 4 * g4 + ii;
          av[ii] = (jl < li) ? bt * __expf(gt - gv.gam[b1][16 * w + jl]) * acc[ii] : 0.f;
        }
        float* ad = Ad[w];  // row-major 16 x 16 block, pitch kAdP
        *reinterpret_cast<float4*>(ad + li * kAdP + 4 * g4) = make_float4(av[0], av[1], av[2], av[3]);
        // Forward substitution on 64 lanes: lane (c = lane/4, k = lane%4) holds rows 4q+k of column c of
        // T_ww; x_m is broadcast inside each quad with DPP. A is strictly lower (zeros on and above the
        // diagonal), so the update needs no row mask.
        const int c = lane >> 2, kq = lane & 3;
        float ar[4][16];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int m4 = 0; m4 < 4; ++m4) {
            const float4 v4 = *reinterpret_cast<const float4*>(ad + (4 * q + kq) * kAdP + 4 * m4);
            ar[q][4 * m4] = v4.x; ar[q][4 * m4 + 1] = v4.y; ar[q][4 * m4 + 2] = v4.z; ar[q][4 * m4 + 3] = v4.w;
          }
        float x[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = (4 * q + kq == c) ? 1.f : 0.f;
#pragma unroll
        for (int m = 0; m < 15; ++m) {
          const float xm = quad_bcast(x[m >> 2], m & 3);
#pragma unroll
          for (int q = 0; q < 4; ++q) x[q] -= ar[q][m] * xm;
        }
        float* tf = &Tf[w >> 1][(16 * (w & 1)) * kTfP + 16 * (w & 1) + c];
        bf16* tb = &Tb[b1][(16 * w) * kCP + 16 * w + c];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * q + kq;
          tf[r * kTfP] = x[q];
          tb[r * kCP] = static_cast<bf16>(r == c ? 0.f : x[q]);
        }
      }
      if (s_on) {  // X = beta V - beta e^gam (K S) -> Xb; kept in fp32 for the identity part of T
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int vv = 16 * nt + li;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int j = 16 * w + 4 * g4 + ii;
            xacc[nt][ii] = gv.bet[b0][j] * (float)Vc[j * kVP + vv] - gv.begam[b0][j] * yacc[nt][ii];
          }
          *reinterpret_cast<bf16x4*>(Xb + vv * kCP + 16 * w + 4 * g4) =
              to_bf16x4(xacc[nt][0], xacc[nt][1], xacc[nt][2], xacc[nt][3]);
        }
      }
    } else {
      const int wz = w - 4;
      // 16 jobs: 6 off-diagonal k.k tiles of chunk i+1 (-> Ao) and 10 k.q tiles of chunk i (-> P)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int job = wz + 4 * jj;
        const bool isq = job >= 6;
        if (isq ? !s_on : !k_on) continue;
        int rb, cb;
        if (!isq) {  // (rb < cb) pairs: (0,1),(0,2),(0,3),(1,2),(1,3),(2,3)
          rb = job < 3 ? 0 : job < 5 ? 1 : 2;
          cb = job < 3 ? job + 1 : job < 5 ? job - 1 : 3;
        } else {  // (rb <= cb) pairs
          const int tj = job - 6;
          rb = tj < 4 ? 0 : tj < 7 ? 1 : tj < 9 ? 2 : 3;
          cb = tj < 4 ? tj : tj < 7 ? tj - 3 : tj < 9 ? tj - 5 : 3;
        }
        const int bb = isq ? b0 : b1;
        const bf16* ka = Kc[bb];
        const bf16* bsrc = isq ? Qc[bb] : Kc[bb];
        bf16x8 fa[KS], fb[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          fa[s] = ld8(ka + (16 * rb + li) * KP + 32 * s + 8 * g4);
          fb[s] = ld8(bsrc + (16 * cb + li) * KP + 32 * s + 8 * g4);
        }
        f32x4 acc{};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = mma(fa[s], fb[s], acc);
        // element (r, c) -> row t = 16cb + li, column j = 16rb + 4g + i
        const int tt = 16 * cb + li, j0 = 16 * rb + 4 * g4;
        const float gt = gv.gam[bb][tt];
        float val[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int j = j0 + ii;
          const float d = __expf(gt - gv.gam[bb][j]);
          val[ii] = (isq ? (j <= tt) : true) ? d * acc[ii] : 0.f;
        }
        if (isq) {
          *reinterpret_cast<bf16x4*>(Pb + tt * kCP + j0) = to_bf16x4(val[0], val[1], val[2], val[3]);
        } else {
          const float bt = gv.bet[bb][tt];
          *reinterpret_cast<float4*>(&Ao[(tt - 16) * kAoP + j0]) = make_float4(bt * val[0], bt * val[1], bt * val[2], bt * val[3]);
        }
      }
      if (s_on) {  // Z = Q S for row tile wz
        const bf16* qb = Qc[b0];
        zacc[0] = f32x4{};
        zacc[1] = f32x4{};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 a = ld8(qb + (16 * wz + li) * KP + 32 * s + 8 * g4);
          const bf16x8 s0 = ld8(Sb + li * KP + 32 * s + 8 * g4);
          const bf16x8 s1 = ld8(Sb + (16 + li) * KP + 32 * s + 8 * g4);
          zacc[0] = mma(a, s0, zacc[0]);
          zacc[1] = mma(a, s1, zacc[1]);
        }
      }
    }
    __syncthreads();

    // ================================================================ phase B
    if (w < 4) {
      if (s_on) {  // Delta = X + (T - I) X for row tile w -> Db, Delta~ hi/lo
        f32x4 dacc[2] = {xacc[0], xacc[1]};
        const bf16* tb = Tb[b0];
        const int ksteps = (w >= 2) ? 2 : 1;  // (T - I) vanishes for j >= t
        for (int s = 0; s < ksteps; ++s) {
          const bf16x8 a = ld8(tb + (16 * w + li) * kCP + 32 * s + 8 * g4);
          const bf16x8 x0 = ld8(Xb + li * kCP + 32 * s + 8 * g4);
          const bf16x8 x1 = ld8(Xb + (16 + li) * kCP + 32 * s + 8 * g4);
          dacc[0] = mma(a, x0, dacc[0]);
          dacc[1] = mma(a, x1, dacc[1]);
        }
        const int tb0 = 16 * w + 4 * g4;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int vv = 16 * nt + li;
          *reinterpret_cast<bf16x4*>(Db + vv * kCP + tb0) = to_bf16x4(dacc[nt][0], dacc[nt][1], dacc[nt][2], dacc[nt][3]);
          bf16x4 hi, lo;
          const float* dl = &gv.dlast[b0][tb0];
          split4(dl[0] * dacc[nt][0], dl[1] * dacc[nt][1], dl[2] * dacc[nt][2], dl[3] * dacc[nt][3], hi, lo);
          *reinterpret_cast<bf16x4*>(DtH + vv * kCP + tb0) = hi;
          *reinterpret_cast<bf16x4*>(DtL + vv * kCP + tb0) = lo;
        }
      }
    } else if (w < 6 && k_on) {  // T 16 -> 32 merges: T_{2q+1,2q} = -T_{2q+1,2q+1} (A_{2q+1,2q} T_{2q,2q})
      // W = A T_{2q,2q} lands in accumulator layout (lane (g, i): rows 4g..4g+3 of column i), which is
      // the B-operand layout of the 16x16x16 MFMA, so the second product takes W from registers.
      const int q = w - 4;
      const float* tq = Tf[q];
      f32x4 acc{};
      {
        float a[4], b[4];
        const float* ar = &Ao[(16 * (2 * q + 1) + li - 16) * kAoP + 32 * q + 4 * g4];
        a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
#pragma unroll
        for (int m = 0; m < 4; ++m) b[m] = tq[(4 * g4 + m) * kTfP + li];
        acc = mma16x3(a, b, acc);
      }
      f32x4 acc2{};
      {
        float a[4];
        const float b[4] = {acc[0], acc[1], acc[2], acc[3]};
        const float* ar = &tq[(16 + li) * kTfP + 16 + 4 * g4];
        a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
        acc2 = mma16x3(a, b, acc2);
      }
      float* tw = &Tf[q][16 * kTfP];
      bf16* tbw = &Tb[b1][(32 * q + 16) * kCP + 32 * q];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        tw[(4 * g4 + ii) * kTfP + li] = -acc2[ii];
        tbw[(4 * g4 + ii) * kCP + li] = static_cast<bf16>(-acc2[ii]);
      }
    }
    __syncthreads();

    // ================================================================ phase C
    if (s_on) {
      if (w >= 4) {  // O = scale (e^gam Z + P Delta) for row tile wz
        const int wz = w - 4;
        f32x4 oacc[2] = {};
        const int ksteps = (wz >= 2) ? 2 : 1;
        for (int s = 0; s < ksteps; ++s) {
          const bf16x8 a = ld8(Pb + (16 * wz + li) * kCP + 32 * s + 8 * g4);
          oacc[0] = mma(a, ld8(Db + li * kCP + 32 * s + 8 * g4), oacc[0]);
          oacc[1] = mma(a, ld8(Db + (16 + li) * kCP + 32 * s + 8 * g4), oacc[1]);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int tt = 16 * wz + 4 * g4 + ii;
          if (tt < len) {
            bf16* orow = og + ((c0 + tt) * p.HV + hv) * VD + vb * kVB + li;
            const float eg = gv.egam[b0][tt];
            orow[0] = static_cast<bf16>(p.scale * (eg * zacc[0][ii] + oacc[0][ii]));
            orow[16] = static_cast<bf16>(p.scale * (eg * zacc[1][ii] + oacc[1][ii]));
          }
        }
      }
      // S' = e^{gam_c} S + K^T Delta~ (hi + lo)
      const float ec = __expf(gv.gam[b0][kC - 1]);
      const bf16* kb = Kc[b0];
#pragma unroll
      for (int u = 0; u < SMAX; ++u) {
        if (u >= s_count) break;
        const int ti = s_first + u, rt = ti >> 1, nt = ti & 1;
        sacc[u] *= ec;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 a = ld8_tr(kb, KP, 32 * s, 16 * rt, lane);
          const int off = (16 * nt + li) * kCP + 32 * s + 8 * g4;
          sacc[u] = mma(a, ld8(DtH + off), sacc[u]);
          sacc[u] = mma(a, ld8(DtL + off), sacc[u]);
        }
      }
    }
    if ((w == 2 || w == 3) && k_on) {  // T 32 -> 64: T[32:64][0:32] = -T[32:64][32:64] (A[32:64][0:32] T[0:32][0:32])
      const int ct = w - 2;  // column block of the result
      f32x4 wacc[2];         // W' tiles (rt, ct), kept in registers as the B operand of the second product
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        wacc[rt] = f32x4{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (ks < ct) continue;  // T[k][c] vanishes for k < c
          float a[4], b[4];
          const float* ar = &Ao[(16 + 16 * rt + li) * kAoP + 16 * ks + 4 * g4];
          a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
#pragma unroll
          for (int m = 0; m < 4; ++m) b[m] = Tf[0][(16 * ks + 4 * g4 + m) * kTfP + 16 * ct + li];
          wacc[rt] = mma16x3(a, b, wacc[rt]);
        }
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        f32x4 acc{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (ks > rt) continue;  // T[32+r][32+k] vanishes for k > r
          float a[4];
          const float b[4] = {wacc[ks][0], wacc[ks][1], wacc[ks][2], wacc[ks][3]};
          const float* ar = &Tf[1][(16 * rt + li) * kTfP + 16 * ks + 4 * g4];
          a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
          acc = mma16x3(a, b, acc);
        }
        bf16* tbw = &Tb[b1][(32 + 16 * rt) * kCP + 16 * ct];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) tbw[(4 * g4 + ii) * kCP + li] = static_cast<bf16>(-acc[ii]);
      }
    }
    if (s_on) {
#pragma unroll
      for (int u = 0; u < SMAX; ++u) {
        if (u >= s_count) break;
        const int ti = s_first + u, kd0 = 16 * (ti >> 1) + 4 * g4, vv = 16 * (ti & 1) + li;
        *reinterpret_cast<bf16x4*>(Sb + vv * KP + kd0) = to_bf16x4(sacc[u][0], sacc[u][1], sacc[u][2], sacc[u][3]);
      }
    }
    __syncthreads();

    // ================================================================ stage chunk i+2 (K/Q/gates), i+1 (V)
    {  // always consume the prefetch registers (zeros past the last chunk) so no load stays pending
      const int64_t cn = bos + (int64_t)(i + 2) * kC;
      stage_kq(b0, i + 2 < nc ? (int)((eos - cn) < kC ? (eos - cn) : kC) : 0);
    }
    stage_v();
    __syncthreads();
  }

  if (p.ht) {
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      if (u >= s_count) break;
      const int ti = s_first + u, kd0 = 16 * (ti >> 1) + 4 * g4, vv = 16 * (ti & 1) + li;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) p.ht[sbase + (int64_t)(kd0 + ii) * VD + vv] = sacc[u][ii];
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


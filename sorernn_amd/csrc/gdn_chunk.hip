// The state kernel of the chunked gated delta rule forward (prefill) for gfx950: bf16 MFMA,
// 64-token chunks, the fp32 state held in MFMA accumulators across the whole sequence. T =
// (I + A)^-1 of every chunk comes from gated_delta_chunk_prep_kernel through the workspace.
//
// Work split: one workgroup (8 waves, two per SIMD) per (sequence, value head, 32-column slice of V).
// The state columns evolve independently, so the slice's state S_b [K x 32] never leaves the
// workgroup. The V/32 slices of one (sequence, head) are placed on the same XCD, so the q/k tiles
// they all read come from one L2.
//
// Per chunk of c <= 64 tokens with gam = in-chunk cumsum of g (sore/model/gdn_ref.py:17-21 in
// chunk form; the algebra is restated in oracle/gdn_oracle.py::_chunk_segment):
//   X     = diag(beta) V - diag(beta exp(gam)) K S              Delta = T X = X + (T - I) X
//   O     = scale (diag(exp(gam)) Q S + P Delta),  P_tj = exp(gam_t - gam_j) q_t.k_j  (j <= t)
//   S'    = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta
//
// Phases per chunk i (one barrier each; SIMD s runs waves s and s + 4):
//   A: waves 0-3 Y = K S (row tile w) -> X;        waves 4-7 Z = Q S (row tile w - 4), O of chunk
//                                                   i-1 to HBM (16-byte stores), V/T loads of i+1.
//   B: waves 0-3 Delta (row tile w), then stage      waves 4-7 P of chunk i+1 (off the chain).
//      K/gates of chunk i+2, load chunk i+3.
//   C: waves 0-3 S' (4 state tiles each);           waves 4-7 O (row tile w - 4) -> LDS, stage
//                                                   V/T of i+1 and Q of i+2, load Q of i+3.
// Loads are issued one iteration before their data is written to LDS, and every LDS slot is
// rewritten only after the phase that last reads it (K and gates: three slots, Q and P: two).
//
// Precision: q/k/v are bf16, so P tiles are exact products with fp32 accumulation. S, X and Delta
// enter MFMA as single bf16; the state update's right operand is split into bf16 hi + lo (two
// MFMAs), which keeps the fp32 final state within 1e-3 relative L2 over 64 chunks.
//
// LDS operand layouts (bf16 rows padded by 8 elements):
//   Kc, Qc [token][key]  natural tiles: A/B operands with the key dim contiguous;
//                        K^T for the state update is read with ds_read_b64_tr_b16.
//   Sb [v][key], Xb/Db/DtH/DtL [v][token], Tb/Pb [t][j]: written from accumulators with 8-byte stores.

#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

struct ChunkParams {
  const void *q, *k, *v, *g, *beta;
  const float* h0;
  void* o;
  float* ht;
  const bf16* tw;  // T - I rows from the prep kernel
  const void* cu;
  const int* order;  // with cu: sequences by length, longest first
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
};

constexpr int kVB = 32;       // value columns per workgroup
constexpr int kNT = 512;      // threads per workgroup (8 waves)
constexpr int kVP = kVB + 8;  // bf16 pitch of the V slice (80 B rows)

// A wave's list of P tiles (rb * 4 + cb each, up to three) packed into one template constant
constexpr int kNoTile = 31;
constexpr int p_tiles(int a, int b, int c) { return a | (b << 5) | (c << 10); }

template <int KD, int VD>
__global__ __launch_bounds__(kNT, 1) void gated_delta_chunk_kernel(ChunkParams p) {
  constexpr int NVB = VD / kVB;
  constexpr int KP = KD + 8;            // bf16 pitch of the q/k tiles
  constexpr int KS = KD / 32;           // MFMA k-steps over the key dim
  constexpr int KCH = KD / 8;           // 16-byte chunks per q/k row
  constexpr int QKPT = kC * KCH / (kNT / 2);  // 16-byte chunks per thread of a q or k tile (half the waves)
  constexpr int SPW = KD / 32;          // state tiles (16 x 16) per wave on waves 0-3

  __shared__ __align__(16) bf16 Kc[3][kC * KP];  // K of chunk c in slot c % 3 (i, i+1, i+2 staged)
  __shared__ __align__(16) bf16 Qc[2][kC * KP];  // Q of chunk c in slot c % 2
  __shared__ __align__(16) bf16 Vc[kC * kVP];    // V slice of chunk i
  __shared__ __align__(16) bf16 Ob[kC * kVP];    // O of chunk i, stored to HBM in the next phase A
  __shared__ __align__(16) bf16 Sb[kVB * KP];
  __shared__ __align__(16) bf16 Tb[kC * kCP];     // T - I of chunk i, A operand [t][j]
  __shared__ __align__(16) bf16 Pb[2][kC * kCP];  // P of chunks i and i+1
  __shared__ __align__(16) bf16 Xb[kVB * kCP];
  __shared__ __align__(16) bf16 Db[kVB * kCP];
  __shared__ __align__(16) bf16 DtH[kVB * kCP];
  __shared__ __align__(16) bf16 DtL[kVB * kCP];
  __shared__ __align__(16) ChunkGates gv[3];      // gate terms of chunk c in slot c % 3

  const int t = threadIdx.x, lane = t & 63, w = t >> 6, g4 = lane >> 4, li = lane & 15;

  // workgroup -> (chain rank k, slice vb) -> (sequence n, value head hv). Workgroups are dispatched
  // in blockIdx order and blockIdx b lands on XCD b % 8: XCD x takes chain ranks x, x + 8, ..., all
  // NVB slices of a chain on one XCD (its q/k tiles are then read from one L2). Chain ranks follow
  // the longest-first sequence order with cu_seqlens, so a grid larger than the machine starts the
  // longest recurrences first.
  const int64_t chains = p.N * p.HV;
  int64_t k_rank;
  int vb;
  if (chains % 8 == 0) {
    const int64_t x = blockIdx.x % 8, j = blockIdx.x / 8;
    k_rank = 8 * (j / NVB) + x;
    vb = (int)(j % NVB);
  } else {
    k_rank = blockIdx.x / NVB;
    vb = (int)(blockIdx.x % NVB);
  }
  const int hv = (int)(k_rank % p.HV);
  const int64_t n = p.order ? (int64_t)p.order[k_rank / p.HV] : k_rank / p.HV;
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
  const float a_log = p.A_log ? p.A_log[hv] : 0.f, dt_b = p.dt_bias ? p.dt_bias[hv] : 0.f;
  const bf16* __restrict__ qg = static_cast<const bf16*>(p.q);
  const bf16* __restrict__ kg = static_cast<const bf16*>(p.k);
  const bf16* __restrict__ vg = static_cast<const bf16*>(p.v);
  bf16* __restrict__ og = static_cast<bf16*>(p.o);
  constexpr int kGateWave = 0;  // loads and scans the gates

  auto chunk_len = [&](int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    return c < nc ? (int)((eos - c0) < kC ? (eos - c0) : kC) : 0;
  };

  // ------------------------------------------------------------------ prefetch registers
  // Waves 0-3 load K/gates of a chunk at the end of phase B and stage them one iteration later
  // (end of the next phase B); waves 4-7 load Q at the end of phase C and V/T at the start of phase
  // A, and stage them at the end of the next phase C. Each prefetch register is consumed at one
  // point only, so no wait for a load in flight is needed anywhere else (rows past the end load as
  // zeros: the load count is fixed).
  // pr holds K rows in waves 0-3 and Q rows in waves 4-7 (one register array for both roles)
  bf16x8 pr[QKPT], pv{}, pt[2];
  uint32_t pgraw = 0, pbraw = 0;
  const int th = t & (kNT / 2 - 1);  // thread index within its half (waves 0-3 or 4-7)
  // Rows u0..u1-1 of this thread's share of a q/k tile. The loads of one tile are issued in three
  // parts at different phases (u in [0, QA), [QA, QB), [QB, QKPT)). All loads go through buffer
  // resources sized to the chunk's valid rows, so rows past the end read as zeros.
  constexpr int QA = QKPT / 2, QB = QKPT * 3 / 4;
  const uint32_t qk_row = (uint32_t)(p.H * KD * 2), v_row = (uint32_t)(p.HV * VD * 2), t_row = (uint32_t)(p.HV * kC * 2);
  auto fetch_rows = [&](bf16x8 (&dst)[QKPT], const bf16* src, int c, int u0, int u1) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const auto rs = make_rsrc(src + (c0 * p.H + h) * KD, (uint32_t)chunk_len(c) * qk_row);
#pragma unroll
    for (int u = 0; u < QKPT; ++u) {
      if (u < u0 || u >= u1) continue;
      const int e = th + u * (kNT / 2), row = e / KCH, c8 = e % KCH;
      dst[u] = buf_load16(rs, row * qk_row + c8 * 16);
    }
  };
  auto stage_rows = [&](const bf16x8 (&src)[QKPT], bf16* dst) {
#pragma unroll
    for (int u = 0; u < QKPT; ++u) {
      const int e = th + u * (kNT / 2), row = e / KCH, c8 = e % KCH;
      *reinterpret_cast<bf16x8*>(&dst[row * KP + c8 * 8]) = l2 ? l2norm_row_chunk<KCH>(src[u]) : src[u];
    }
  };
  auto fetch_k = [&](int c, int u0, int u1) {  // waves 0-3: K rows of chunk c (and with u0 == 0 its gates)
    fetch_rows(pr, kg, c, u0, u1);
    if (u0 > 0) return;
    const int64_t c0 = bos + (int64_t)c * kC;
    const uint32_t gb = (uint32_t)(p.HV * dtype_bytes(p.dg)), bb = (uint32_t)(p.HV * dtype_bytes(p.db));
    const uint32_t len = (uint32_t)chunk_len(c);
    const auto rg = make_rsrc(static_cast<const char*>(p.g) + (c0 * p.HV + hv) * dtype_bytes(p.dg), len * gb);
    const auto rb = make_rsrc(static_cast<const char*>(p.beta) + (c0 * p.HV + hv) * dtype_bytes(p.db), len * bb);
    pgraw = buf_load_raw32(rg, lane * gb, p.dg);
    pbraw = buf_load_raw32(rb, lane * bb, p.db);
  };
  auto stage_gates = [&](int c) {  // wave kGateWave: gate slot c % 3
    if (w == kGateWave)
      chunk_gates_from_raw(gv[c % 3], pgraw, pbraw, p.dg, p.db, chunk_len(c), p.flags, a_log, dt_b, lane);
  };
  auto fetch_vt = [&](int c) {  // waves 4-7: V slice and T - I rows of chunk c
    const int64_t c0 = bos + (int64_t)c * kC;
    const uint32_t len = (uint32_t)chunk_len(c);
    const auto rv = make_rsrc(vg + (c0 * p.HV + hv) * VD + vb * kVB, len * v_row);
    pv = buf_load16(rv, (th >> 2) * v_row + (th & 3) * 16);
    const auto rt = make_rsrc(p.tw + (c0 * p.HV + hv) * kC, len * t_row);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = th + u * (kNT / 2);
      pt[u] = buf_load16(rt, (e >> 3) * t_row + (e & 7) * 16);
    }
  };
  auto stage_vt = [&]() {  // waves 4-7
    *reinterpret_cast<bf16x8*>(Vc + (th >> 2) * kVP + (th & 3) * 8) = pv;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = th + u * (kNT / 2);
      *reinterpret_cast<bf16x8*>(Tb + (e >> 3) * kCP + (e & 7) * 8) = pt[u];
    }
  };
  auto store_o = [&](int c) {  // waves 4-7: O of chunk c from Ob to HBM, 16 bytes per thread
    const int64_t c0 = bos + (int64_t)c * kC;
    const auto ro = make_rsrc(og + (c0 * p.HV + hv) * VD + vb * kVB, (uint32_t)chunk_len(c) * v_row);
    const int row = th >> 2, c8 = th & 3;
    buf_store16(*reinterpret_cast<const bf16x8*>(Ob + row * kVP + c8 * 8), ro, row * v_row + c8 * 16);
  };

  // P of the chunk in buffer `buf`: tile (rb, cb), rb <= cb, holds element (j = 16rb + 4g + i,
  // t = 16cb + li) = exp(gam_t - gam_j) k_j.q_t for j <= t. The 10 tiles are dealt to waves 4-7 as
  // 3, 3, 2, 2 (code: up to three 5-bit fields rb * 4 + cb, kNoTile = none), so with Delta on
  // waves 0-3 every SIMD issues 12-14 MFMAs in phase B.
  auto p_job = [&](auto code_c, const bf16* kb, const bf16* qb, bf16* pw, const ChunkGates& gs) {
    constexpr int code = decltype(code_c)::value;
    bf16x8 fa[3][KS], fb[3][KS];
    float gtc[3];
    float4 gjs[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int tc = (code >> (5 * q)) & 31;
      if (tc == kNoTile) continue;
      const int rb = tc >> 2, cb = tc & 3;
      gtc[q] = gs.gam[16 * cb + li];
      gjs[q] = ld4f(&gs.gam[16 * rb + 4 * g4]);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        fa[q][s] = ld8(kb + (16 * rb + li) * KP + 32 * s + 8 * g4);
        fb[q][s] = ld8(qb + (16 * cb + li) * KP + 32 * s + 8 * g4);
      }
    }
    f32x4 pacc[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      if (((code >> (5 * q)) & 31) == kNoTile) continue;
      pacc[q] = f32x4{};
#pragma unroll
      for (int s = 0; s < KS; ++s) pacc[q] = mma(fa[q][s], fb[q][s], pacc[q]);
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int tc = (code >> (5 * q)) & 31;
      if (tc == kNoTile) continue;
      const int rb = tc >> 2, cb = tc & 3;
      const int tt = 16 * cb + li, j0 = 16 * rb + 4 * g4;
      const float gt = gtc[q];
      const float dd[4] = {__expf(gt - gjs[q].x), __expf(gt - gjs[q].y), __expf(gt - gjs[q].z), __expf(gt - gjs[q].w)};
      float val[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) val[ii] = (cb > rb || j0 + ii <= tt) ? dd[ii] * pacc[q][ii] : 0.f;
      *reinterpret_cast<bf16x4*>(pw + tt * kCP + j0) = to_bf16x4(val[0], val[1], val[2], val[3]);
    }
  };
  auto run_p_side = [&](int c) {  // waves 4-7: P of chunk c into Pb[c % 2]
    const bf16* kb = Kc[c % 3];
    const bf16* qb = Qc[c & 1];
    bf16* pw = Pb[c & 1];
    const ChunkGates& gs = gv[c % 3];
    switch (w) {  // tiles (0,0) (0,1) (0,2) | (0,3) (1,1) (1,2) | (1,3) (2,2) | (2,3) (3,3)
      case 4: p_job(std::integral_constant<int, p_tiles(0, 1, 2)>{}, kb, qb, pw, gs); break;
      case 5: p_job(std::integral_constant<int, p_tiles(3, 5, 6)>{}, kb, qb, pw, gs); break;
      case 6: p_job(std::integral_constant<int, p_tiles(7, 10, kNoTile)>{}, kb, qb, pw, gs); break;
      default: p_job(std::integral_constant<int, p_tiles(11, 15, kNoTile)>{}, kb, qb, pw, gs); break;
    }
  };

  // P is causally lower: its tiles above the diagonal stay zero for the whole run
  for (int e = t; e < kC * kCP / 8; e += kNT) {
    reinterpret_cast<bf16x8*>(Pb[0])[e] = bf16x8{};
    reinterpret_cast<bf16x8*>(Pb[1])[e] = bf16x8{};
  }

  // Loop-carried accumulators share one register array: waves 0-3 hold their state tiles in
  // racc[0 .. SPW) and X of their row tile in racc[SPW .. SPW+2); waves 4-7 hold Z in racc[0..1].
  f32x4 racc[SPW + 2];
  const int s_first = w * SPW;  // state tiles ti = s_first + u: row tile ti / 2, column tile ti % 2
  const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVB;
#pragma unroll
  for (int u = 0; u < SPW; ++u) {
    if (w >= 4) break;
    const int ti = s_first + u, kd0 = 16 * (ti >> 1) + 4 * g4, vv = 16 * (ti & 1) + li;
#pragma unroll
    for (int i = 0; i < 4; ++i) racc[u][i] = p.h0 ? p.h0[sbase + (int64_t)(kd0 + i) * VD + vv] : 0.f;
    *reinterpret_cast<bf16x4*>(Sb + vv * KP + kd0) = to_bf16x4(racc[u][0], racc[u][1], racc[u][2], racc[u][3]);
  }

  // prologue: K/Q/gates of chunks 0 and 1, V/T of chunk 0 staged, K/Q of chunk 2 in flight, P of chunk 0
  if (w < 4) {
    fetch_k(0, 0, QKPT);
    stage_rows(pr, Kc[0]);
    stage_gates(0);
    fetch_k(1, 0, QKPT);
    stage_rows(pr, Kc[1]);
    stage_gates(1);
    fetch_k(2, 0, QB);  // the rest in phase A of chunk 0
  } else {
    fetch_rows(pr, qg, 0, 0, QKPT);
    stage_rows(pr, Qc[0]);
    fetch_rows(pr, qg, 1, 0, QKPT);
    stage_rows(pr, Qc[1]);
    fetch_rows(pr, qg, 2, 0, QA);  // the rest in phases A and B of chunk 0
    fetch_vt(0);
    stage_vt();
  }
  __syncthreads();
  if (w >= 4 && nc > 0) run_p_side(0);
  __syncthreads();

  // Operands that do not depend on the previous phase are read from LDS one phase early, so each
  // phase starts with only its state-dependent reads outstanding: fpre (K rows of the Y tile in
  // waves 0-3, Q rows of the Z tile in waves 4-7) at the end of phase C for the next chunk, the T
  // fragments of Delta at the end of phase A, the K^T fragments of the state update at the end of B.
  constexpr int NRT = SPW / 2;  // row tiles of K in a wave's state tiles
  bf16x8 fpre[KS], tpre[2], ktr[NRT][2];
  auto preload_f = [&](int c) {
    const bf16* src = (w < 4) ? Kc[c % 3] + (16 * w + li) * KP : Qc[c & 1] + (16 * (w - 4) + li) * KP;
#pragma unroll
    for (int s = 0; s < KS; ++s) fpre[s] = ld8(src + 32 * s + 8 * g4);
  };
  preload_f(0);

  for (int i = 0; i < nc; ++i) {
    const int ks = i % 3, qs = i & 1;  // K/gate slot and Q/P slot of chunk i
    const ChunkGates& G0 = gv[ks];

    // ================================================================ phase A
    if (w < 4) {  // Y = K S for row tile w, then X = beta V - beta e^gam Y -> Xb (fp32 copy kept)
      fetch_k(i + 2, QB, QKPT);
      const int r = w, j0 = 16 * r + 4 * g4;
      float vx[2][4];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) vx[nt][ii] = (float)Vc[(j0 + ii) * kVP + 16 * nt + li];
      const float4 bj = ld4f(&G0.bet[j0]), bgj = ld4f(&G0.begam[j0]);
      bf16x8 sf[2][KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sf[0][s] = ld8(Sb + li * KP + 32 * s + 8 * g4);
        sf[1][s] = ld8(Sb + (16 + li) * KP + 32 * s + 8 * g4);
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x4 yacc[2] = {};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        yacc[0] = mma(fpre[s], sf[0][s], yacc[0]);
        yacc[1] = mma(fpre[s], sf[1][s], yacc[1]);
      }
      const float bjv[4] = {bj.x, bj.y, bj.z, bj.w}, bgjv[4] = {bgj.x, bgj.y, bgj.z, bgj.w};
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) racc[SPW + nt][ii] = bjv[ii] * vx[nt][ii] - bgjv[ii] * yacc[nt][ii];
        *reinterpret_cast<bf16x4*>(Xb + (16 * nt + li) * kCP + j0) =
            to_bf16x4(racc[SPW + nt][0], racc[SPW + nt][1], racc[SPW + nt][2], racc[SPW + nt][3]);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) tpre[s] = ld8(Tb + (16 * w + li) * kCP + 32 * s + 8 * g4);
    } else {  // V/T of chunk i+1 requested; Z = Q S for row tile w - 4 (kept for O); O of chunk i-1 out
      fetch_vt(i + 1);
      fetch_rows(pr, qg, i + 2, QA, QB);
      const int r = w - 4;
      bf16x8 sf[2][KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sf[0][s] = ld8(Sb + li * KP + 32 * s + 8 * g4);
        sf[1][s] = ld8(Sb + (16 + li) * KP + 32 * s + 8 * g4);
      }
      __builtin_amdgcn_sched_barrier(0);
      racc[0] = f32x4{};
      racc[1] = f32x4{};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        racc[0] = mma(fpre[s], sf[0][s], racc[0]);
        racc[1] = mma(fpre[s], sf[1][s], racc[1]);
      }
      if (i > 0) store_o(i - 1);
    }
    __syncthreads();

    // ================================================================ phase B
    if (w < 4) {  // Delta = X + (T - I) X for row tile w -> Db, Delta~ = exp(gam_c - gam) Delta hi/lo
      f32x4 dacc[2] = {racc[SPW], racc[SPW + 1]};
      const int ksteps = (w >= 2) ? 2 : 1;  // (T - I) vanishes for j >= t
      for (int s = 0; s < ksteps; ++s) {
        const bf16x8 a = tpre[s];
        const bf16x8 x0 = ld8(Xb + li * kCP + 32 * s + 8 * g4);
        const bf16x8 x1 = ld8(Xb + (16 + li) * kCP + 32 * s + 8 * g4);
        dacc[0] = mma(a, x0, dacc[0]);
        dacc[1] = mma(a, x1, dacc[1]);
      }
      const int tb0 = 16 * w + 4 * g4;
      const float4 dl = ld4f(&G0.dlast[tb0]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int vv = 16 * nt + li;
        *reinterpret_cast<bf16x4*>(Db + vv * kCP + tb0) = to_bf16x4(dacc[nt][0], dacc[nt][1], dacc[nt][2], dacc[nt][3]);
        bf16x4 hi, lo;
        split4(dl.x * dacc[nt][0], dl.y * dacc[nt][1], dl.z * dacc[nt][2], dl.w * dacc[nt][3], hi, lo);
        *reinterpret_cast<bf16x4*>(DtH + vv * kCP + tb0) = hi;
        *reinterpret_cast<bf16x4*>(DtL + vv * kCP + tb0) = lo;
      }
      // K/gates of chunk i+2 into their slots (last read by chunk i-1), then the first loads of chunk i+3
      stage_rows(pr, Kc[(i + 2) % 3]);
      stage_gates(i + 2);
      fetch_k(i + 3, 0, QA);
#pragma unroll
      for (int u = 0; u < NRT; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s) ktr[u][s] = ld8_tr(Kc[ks], KP, 32 * s, 16 * (NRT * w + u), lane);
    } else {  // P of chunk i+1, off the state chain
      fetch_rows(pr, qg, i + 2, QB, QKPT);
      if (i + 1 < nc) run_p_side(i + 1);
    }
    __syncthreads();

    // ================================================================ phase C
    if (w >= 4) {  // O = scale (e^gam Z + P Delta) for row tile r -> Ob; V/T of chunk i+1 staged
      const int r = w - 4;
      f32x4 oacc[2] = {};
      const int ksteps = (r >= 2) ? 2 : 1;
      for (int s = 0; s < ksteps; ++s) {
        const bf16x8 a = ld8(Pb[qs] + (16 * r + li) * kCP + 32 * s + 8 * g4);
        oacc[0] = mma(a, ld8(Db + li * kCP + 32 * s + 8 * g4), oacc[0]);
        oacc[1] = mma(a, ld8(Db + (16 + li) * kCP + 32 * s + 8 * g4), oacc[1]);
      }
      const float4 eg = ld4f(&G0.egam[16 * r + 4 * g4]);
      const float egv[4] = {eg.x, eg.y, eg.z, eg.w};
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int tt = 16 * r + 4 * g4 + ii;
        Ob[tt * kVP + li] = static_cast<bf16>(p.scale * (egv[ii] * racc[0][ii] + oacc[0][ii]));
        Ob[tt * kVP + 16 + li] = static_cast<bf16>(p.scale * (egv[ii] * racc[1][ii] + oacc[1][ii]));
      }
      stage_vt();                 // V_i was last read in phase A, T_i in phase B
      stage_rows(pr, Qc[qs]);     // Q of chunk i+2 (Q_i was last read by Z in phase A)
      fetch_rows(pr, qg, i + 3, 0, QA);
    } else {  // S' = e^{gam_c} S + K^T Delta~ (hi + lo) for this wave's state tiles
      fetch_k(i + 3, QA, QB);
      const float ec = __expf(G0.gam[kC - 1]);
#pragma unroll
      for (int u = 0; u < SPW; ++u) {
        const int ti = s_first + u, nt = ti & 1;
        racc[u] *= ec;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 a = ktr[u >> 1][s];  // row tile ti / 2 = s_first / 2 + u / 2
          const int off = (16 * nt + li) * kCP + 32 * s + 8 * g4;
          racc[u] = mma(a, ld8(DtH + off), racc[u]);
          racc[u] = mma(a, ld8(DtL + off), racc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < SPW; ++u) {
        const int ti = s_first + u, kd0 = 16 * (ti >> 1) + 4 * g4, vv = 16 * (ti & 1) + li;
        *reinterpret_cast<bf16x4*>(Sb + vv * KP + kd0) = to_bf16x4(racc[u][0], racc[u][1], racc[u][2], racc[u][3]);
      }
    }
    if (i + 1 < nc) preload_f(i + 1);  // K_{i+1} was staged in phase B of chunk i-1, Q_{i+1} in phase C
    __syncthreads();
  }
  if (w >= 4 && nc > 0) store_o(nc - 1);

  if (p.ht && w < 4) {
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
      const int ti = s_first + u, kd0 = 16 * (ti >> 1) + 4 * g4, vv = 16 * (ti & 1) + li;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) p.ht[sbase + (int64_t)(kd0 + ii) * VD + vv] = racc[u][ii];
    }
  }
}

}  // namespace gdn

using namespace gdn;

extern "C" size_t gdn_chunk_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t N, int varlen) {
  if (B <= 0 || T < 0 || HV <= 0 || N <= 0) return 0;
  size_t bytes = (size_t)chunk_t_bytes(B * T, HV);
  if (varlen) bytes += (size_t)(align256((N + 1) * 4) + align256(N * 4));
  return bytes;
}

extern "C" int gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                             const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                             int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                             int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                             const float* A_log, const float* dt_bias, void* workspace, size_t workspace_bytes,
                             void* stream) {
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
  const size_t need = gdn_chunk_workspace_size(B, T, HV, N, cu_seqlens != nullptr);
  if (need > 0 && (!workspace || workspace_bytes < need)) {
    gdn_internal_set_error("gdn_chunk_fwd: workspace of %zu bytes needed (got %zu)", need,
                           workspace ? workspace_bytes : (size_t)0);
    return GDN_ERR_INVALID;
  }
  if (T == 0) return GDN_OK;
  const int64_t blocks = N * HV * (V / kVB);
  if (blocks > 0x7fffffff) {
    gdn_internal_set_error("gdn_chunk_fwd: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cu_i32 = (flags & GDN_FLAG_CU_INT32) ? 1 : 0;
  bf16* tw = static_cast<bf16*>(workspace);
  char* const ws = static_cast<char*>(workspace);
  const int* chunk_first = cu_seqlens ? reinterpret_cast<const int*>(ws + chunk_t_bytes(B * T, HV)) : nullptr;
  const int* order =
      cu_seqlens ? reinterpret_cast<const int*>(ws + chunk_t_bytes(B * T, HV) + align256((N + 1) * 4)) : nullptr;
  ChunkPrepParams pp{k, g, beta, tw, cu_seqlens, chunk_first, order, cu_i32, T, H, HV, N, g_dtype, beta_dtype, flags,
                     A_log, dt_bias};
  const int rc = launch_chunk_prep(pp, B, K, s);
  if (rc != GDN_OK) return rc;
  ChunkParams p{q, k, v, g, beta, initial_state, o, final_state, tw, cu_seqlens, order, cu_i32, T, H, HV, N,
                g_dtype, beta_dtype, scale, flags, A_log, dt_bias};
  dim3 grid((unsigned)blocks), block(kNT);
  if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 128>), grid, block, 0, s, p);
  else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 64>), grid, block, 0, s, p);
  else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 64>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 128>), grid, block, 0, s, p);
  return gdn_internal_check_launch("gated_delta_chunk_kernel");
}

// The state kernel of the chunked gated delta rule forward (prefill) for gfx950: bf16 MFMA,
// 64-token chunks, the fp32 state held in MFMA accumulators across the whole sequence. T =
// (I + A)^-1 of every chunk comes from gated_delta_chunk_prep_kernel through the workspace.
//
// Per chunk of c <= 64 tokens with gam = in-chunk cumsum of g (sore/model/gdn_ref.py:17-21 in
// chunk form; the algebra is restated in oracle/gdn_oracle.py::_chunk_segment):
//   X     = diag(beta) V - diag(beta exp(gam)) K S              Delta = T X = X + (T - I) X
//   O     = scale (diag(exp(gam)) Q S + P Delta),  P_tj = exp(gam_t - gam_j) q_t.k_j  (j <= t)
//   S'    = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta
//
// Work split: one workgroup of 8 waves per (sequence, value head, 32-column slice of V); the V/32
// slices of one (sequence, head) sit on one XCD, so the tiles they all read come from one L2.
//   State waves 0 and 1 each own 16 state columns, S_b [K x 16] in fp32 accumulators, and run the
//   whole recurrence of their columns: every operand that depends on the state (S itself, X,
//   Delta, Delta~) is an accumulator fragment used in place as the next MFMA's operand, so the
//   state never passes through LDS. Per chunk: Y = K S, X, Delta, O^T = scale(e^gam Z^T +
//   Delta^T P^T), the hi/lo state update, then Z^T = S^T Q^T of the next chunk (76 MFMAs).
//   Helper waves 2-7 stage the chunk-wide operands one chunk ahead: q/k rows (waves 4-7, L2-norm
//   when asked), T - I rows and the V slice (waves 2-3), gate terms (wave 2), the scaled P of the
//   next chunk (waves 2, 3, 6, 7 on SIMDs 2 and 3), and store O of the previous chunk (waves 4-7).
// One barrier per chunk separates the two sides.
//
// Fragment layouts (16x16x32 MFMA, lane (g, i), element r = 0..3 of an accumulator):
//   S tile a = 2s + h (s = 32-deep key step): row 4g + r is key 32s + 8g + 4h + r, so the pair
//     (S_2s, S_2s+1) in bf16 is the B operand of K S (keys 32s + 8g..+7) and the A operand of S^T Q^T;
//     the K^T operand of the update reads K columns in that order (ld8_tr_pair).
//   Y, X, Delta tile b: rows 16b + 4g + r (tokens), column i; pairs (2u, 2u+1) contract over the
//     tokens 32u + 4g + r and 32u + 16 + 4g + r, which is the column order of T - I and P (tok_col).
//   Z^T, O^T tile tb: row 4g + r is the wave's value column, column i the token 16tb + i.
//
// Precision: q/k/v are bf16, so P tiles are exact products with fp32 accumulation. S, X and Delta
// enter MFMA as single bf16; the state update's right operand is split into bf16 hi + lo (two
// MFMAs), which keeps the fp32 final state within 1e-3 relative L2 over 64 chunks.
//
// LDS: K (3 slots), Q (2 slots), T - I, P, V and O (2 slots each), gate terms (3 slots).

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

constexpr int kVB = 32;       // value columns per workgroup (two state waves of 16)
constexpr int kNT = 512;      // threads per workgroup (8 waves)
constexpr int kVP = kVB + 8;  // bf16 pitch of the V and O slices (80 B rows)

template <int KD, int VD>
__global__ __launch_bounds__(kNT, 1) void gated_delta_chunk_kernel(ChunkParams p) {
  constexpr int NVB = VD / kVB;
  constexpr int KP = KD + 8;                  // bf16 pitch of the q/k tiles
  constexpr int KS = KD / 32;                 // MFMA k-steps over the key dim
  constexpr int KT = KD / 16;                 // 16-row state tiles
  constexpr int KCH = KD / 8;                 // 16-byte chunks per q/k row
  constexpr int QKPT = kC * KCH / 256;        // 16-byte chunks per thread of a q or k tile (waves 4-7)

  __shared__ __align__(16) bf16 Kc[3][kC * KP];   // K of chunk c in slot c % 3
  __shared__ __align__(16) bf16 Qc[2][kC * KP];   // Q of chunk c in slot c % 2
  __shared__ __align__(16) bf16 Tb[2][kC * kCP];  // T - I of chunk c in slot c % 2 (tok_col columns)
  __shared__ __align__(16) bf16 Pb[2][kC * kCP];  // scale * P of chunk c in slot c % 2 (tok_col columns)
  __shared__ __align__(16) bf16 Vc[2][kC * kVP];  // V slice of chunk c in slot c % 2
  __shared__ __align__(16) bf16 Ob[2][kC * kVP];  // O of chunk c, stored to HBM during chunk c + 1
  __shared__ __align__(16) ChunkGates gv[3];      // gate terms of chunk c in slot c % 3

  // w is read back as a scalar: the compiler then treats the role branches as wave-uniform
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;

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

  auto chunk_len = [&](int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    return c < nc ? (int)((eos - c0) < kC ? (eos - c0) : kC) : 0;
  };

  // ------------------------------------------------------------------ helper-side staging
  // Each helper loads a chunk's operands into registers one chunk before it writes them to LDS, so
  // the loads have a whole chunk step to land. All loads go through buffer resources sized to the
  // chunk's valid rows: rows past the end (and chunks past the sequence) read as zeros.
  const uint32_t qk_row = (uint32_t)(p.H * KD * 2), v_row = (uint32_t)(p.HV * VD * 2), t_row = (uint32_t)(p.HV * kC * 2);
  const int th4 = t & 255;         // waves 4-7: q/k rows, O store
  const int th2 = (t - 128) & 127;  // waves 2-3: T - I rows, V slice
  // Loop-carried registers, one array for both sides (a wave uses one role only):
  //   state waves: R[0, KT) = S tiles, R[KT, KT+4) = Z^T tiles, R[KT+4, KT+4+KS) = S pairs in bf16,
  //                R[KT+4+KS, KT+4+3KS) = the K row fragments of the next Y = K S for its first
  //                half of key steps (read ahead across the barrier);
  //   waves 4-7:   R[0, QKPT) = k rows, R[QKPT, 2 QKPT) = q rows in flight;
  //   waves 2-3:   R[0, 4) = T - I rows, R[4, 6) = V rows in flight.
  constexpr int NR = KT + 4 + 3 * KS;
  constexpr int KSH = KS / 2;  // key steps of Y whose K fragments are read ahead
  static_assert(2 * QKPT <= NR && 6 <= NR, "register roles");
  f32x4 R[NR];
  uint32_t pgraw = 0, pbraw = 0;
  // The helpers' per-thread offsets are computed from `tq` (th4 or th2 passed through an empty asm
  // inside the loop), so they are rebuilt in the helper branch each step instead of being hoisted
  // out of the loop into registers that would stay live through the state waves' code.
  // Thread tq of waves 4-7 handles the 16-byte chunks tq + 256u of a q/k tile: row tq / KCH + u (256
  // / KCH), chunk tq % KCH.
  auto fetch_rows = [&](int r0, const bf16* src, int c, int tq) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const auto rs = make_rsrc(src + (c0 * p.H + h) * KD, (uint32_t)chunk_len(c) * qk_row);
    const uint32_t base = (uint32_t)(tq / KCH) * qk_row + (uint32_t)(tq % KCH) * 16;
#pragma unroll
    for (int u = 0; u < QKPT; ++u)
      R[r0 + u] = __builtin_bit_cast(f32x4, buf_load16(rs, base + (uint32_t)(u * (256 / KCH)) * qk_row));
  };
  auto stage_rows = [&](int r0, bf16* dst, int tq) {
    bf16* const d0 = dst + (tq / KCH) * KP + (tq % KCH) * 8;
#pragma unroll
    for (int u = 0; u < QKPT; ++u) {
      const bf16x8 x = __builtin_bit_cast(bf16x8, R[r0 + u]);
      *reinterpret_cast<bf16x8*>(d0 + u * (256 / KCH) * KP) = l2 ? l2norm_row_chunk<KCH>(x) : x;
    }
  };
  // Thread tq of waves 2-3: T - I chunks tq + 128u (row tq / 8 + 16u, 8 chunks of 16 B per row)
  // and V-slice chunks tq + 128u (row tq / 4 + 32u, 4 chunks per row).
  auto fetch_tv = [&](int c, int tq) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const uint32_t len = (uint32_t)chunk_len(c);
    const auto rt = make_rsrc(p.tw + (c0 * p.HV + hv) * kC, len * t_row);
    const uint32_t bt = (uint32_t)(tq >> 3) * t_row + (uint32_t)(tq & 7) * 16;
#pragma unroll
    for (int u = 0; u < 4; ++u) R[u] = __builtin_bit_cast(f32x4, buf_load16(rt, bt + (uint32_t)(16 * u) * t_row));
    const auto rv = make_rsrc(vg + (c0 * p.HV + hv) * VD + vb * kVB, len * v_row);
    const uint32_t bv = (uint32_t)(tq >> 2) * v_row + (uint32_t)(tq & 3) * 16;
#pragma unroll
    for (int u = 0; u < 2; ++u) R[4 + u] = __builtin_bit_cast(f32x4, buf_load16(rv, bv + (uint32_t)(32 * u) * v_row));
  };
  auto stage_tv = [&](int slot, int tq) {
    bf16* const t0 = Tb[slot] + (tq >> 3) * kCP + (tq & 7) * 8;
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<f32x4*>(t0 + 16 * u * kCP) = R[u];
    bf16* const v0 = Vc[slot] + (tq >> 2) * kVP + (tq & 3) * 8;
#pragma unroll
    for (int u = 0; u < 2; ++u) *reinterpret_cast<f32x4*>(v0 + 32 * u * kVP) = R[4 + u];
  };
  auto fetch_gates = [&](int c) {  // wave 2, lane = token
    const int64_t c0 = bos + (int64_t)c * kC;
    const uint32_t gb = (uint32_t)(p.HV * dtype_bytes(p.dg)), bb = (uint32_t)(p.HV * dtype_bytes(p.db));
    const uint32_t len = (uint32_t)chunk_len(c);
    const auto rg = make_rsrc(static_cast<const char*>(p.g) + (c0 * p.HV + hv) * dtype_bytes(p.dg), len * gb);
    const auto rb = make_rsrc(static_cast<const char*>(p.beta) + (c0 * p.HV + hv) * dtype_bytes(p.db), len * bb);
    pgraw = buf_load_raw32(rg, lane * gb, p.dg);
    pbraw = buf_load_raw32(rb, lane * bb, p.db);
  };
  auto stage_gates = [&](int c) {
    chunk_gates_from_raw(gv[c % 3], pgraw, pbraw, p.dg, p.db, chunk_len(c), p.flags, a_log, dt_b, lane);
  };
  auto store_o = [&](int c, int tq) {  // waves 4-7: O of chunk c from Ob to HBM, 16 bytes per thread
    const int64_t c0 = bos + (int64_t)c * kC;
    const auto ro = make_rsrc(og + (c0 * p.HV + hv) * VD + vb * kVB, (uint32_t)chunk_len(c) * v_row);
    const int row = tq >> 2, c8 = tq & 3;
    buf_store16(*reinterpret_cast<const bf16x8*>(&Ob[c & 1][row * kVP + c8 * 8]), ro, row * v_row + c8 * 16);
  };

  // scale * P^T of chunk c for key-row tiles JA..JA+JN-1 and query-row tiles TA..TA+TN-1 (tiles
  // with jt <= tt only): element (j = 16jt + 4g + r, t = 16tt + i), stored at Pb[t][tok_col(j)].
  // Waves 2, 3, 6, 7 (SIMDs 2 and 3) take the 2x2, 2x2, 2x1 and 2x1 tile blocks of the lower triangle.
  auto p_job = [&](auto ja_c, auto jn_c, auto ta_c, auto tn_c, int c, int ln) {
    const int li = ln & 15, g4 = ln >> 4;
    constexpr int JA = decltype(ja_c)::value, JN = decltype(jn_c)::value;
    constexpr int TA = decltype(ta_c)::value, TN = decltype(tn_c)::value;
    const bf16* kb = Kc[c % 3];
    const bf16* qb = Qc[c & 1];
    bf16* pw = Pb[c & 1];
    const ChunkGates& gs = gv[c % 3];
    f32x4 acc[JN][TN];
#pragma unroll
    for (int a = 0; a < JN; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 fk[JN], fq[TN];
#pragma unroll
      for (int a = 0; a < JN; ++a) fk[a] = ld8(kb + (16 * (JA + a) + li) * KP + 32 * s + 8 * g4);
#pragma unroll
      for (int b = 0; b < TN; ++b) fq[b] = ld8(qb + (16 * (TA + b) + li) * KP + 32 * s + 8 * g4);
#pragma unroll
      for (int a = 0; a < JN; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          if (JA + a <= TA + b) acc[a][b] = mma(fk[a], fq[b], acc[a][b]);
    }
#pragma unroll
    for (int a = 0; a < JN; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        const int jt = JA + a, tt_ = TA + b;
        if (jt > tt_) continue;
        const int tt = 16 * tt_ + li, j0 = 16 * jt + 4 * g4;
        const float gt = gs.gam[tt];
        const float4 gj = ld4f(&gs.gam[j0]);
        const float gjv[4] = {gj.x, gj.y, gj.z, gj.w};
        float val[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = (jt < tt_ || j0 + r <= tt) ? p.scale * __expf(gt - gjv[r]) * acc[a][b][r] : 0.f;
        *reinterpret_cast<bf16x4*>(pw + tt * kCP + tok_col(j0)) = to_bf16x4(val[0], val[1], val[2], val[3]);
      }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  auto run_p_side = [&](int c, int ln) {
    switch (w) {
      case 2: p_job(I0{}, I2{}, I0{}, I2{}, c, ln); break;   // (0,0) (0,1) (1,1)
      case 3: p_job(I2{}, I2{}, I2{}, I2{}, c, ln); break;   // (2,2) (2,3) (3,3)
      case 6: p_job(I0{}, I2{}, I2{}, I1{}, c, ln); break;   // (0,2) (1,2)
      case 7: p_job(I0{}, I2{}, I3{}, I1{}, c, ln); break;   // (0,3) (1,3)
      default: break;
    }
  };

  // ------------------------------------------------------------------ state-side registers
  const int sw = w & 1;  // state wave 0 or 1: value columns 16 sw .. 16 sw + 15 of the slice
  // S tile a = R[a]; Z^T = S^T Q^T of the current chunk, tile tb = R[KT + tb] (value column 4g + r,
  // token 16tb + i); (S_2s, S_2s+1) in bf16 = R[KT + 4 + s]
  f32x4* const S = R;
  f32x4* const Zt = R + KT;
  auto sb = [&](int s) { return __builtin_bit_cast(bf16x8, R[KT + 4 + s]); };
  const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVB + 16 * sw;
  auto make_sb = [&]() {
#pragma unroll
    for (int s = 0; s < KS; ++s) R[KT + 4 + s] = __builtin_bit_cast(f32x4, pack8(S[2 * s], S[2 * s + 1]));
  };
  // K row fragments of Y = K S for chunk c, key steps s < KSH (row tile b), read ahead into R
  f32x4* const KF = R + KT + 4 + KS;
  auto load_kf = [&](int c) {
    const bf16* kb = Kc[c % 3];
#pragma unroll
    for (int s = 0; s < KSH; ++s)
#pragma unroll
      for (int b = 0; b < 4; ++b) KF[4 * s + b] = __builtin_bit_cast(f32x4, ld8(kb + (16 * b + li) * KP + 32 * s + 8 * g4));
  };
  // Each phase of the state step issues the LDS reads of the next phase before its own MFMAs, and
  // the scheduler may not move instructions across the phase boundaries: LDS reads complete in
  // order, so every phase finds its operands arrived or in flight instead of starting a round trip.
  auto phase = [] { __builtin_amdgcn_sched_barrier(0); };

  // ------------------------------------------------------------------ prologue
  // P is causally lower: its tiles above the diagonal stay zero for the whole run
  for (int e = t; e < kC * kCP / 8; e += kNT) {
    reinterpret_cast<bf16x8*>(Pb[0])[e] = bf16x8{};
    reinterpret_cast<bf16x8*>(Pb[1])[e] = bf16x8{};
  }
  if (w < 2) {
#pragma unroll
    for (int a = 0; a < KT; ++a) {
      const int kd0 = 32 * (a >> 1) + 8 * g4 + 4 * (a & 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) S[a][r] = p.h0 ? p.h0[sbase + (int64_t)(kd0 + r) * VD + li] : 0.f;
    }
    make_sb();
  } else if (w >= 4) {  // K/Q of chunks 0 and 1 staged, chunk 2 in flight
    fetch_rows(0, kg, 0, th4);
    fetch_rows(QKPT, qg, 0, th4);
    stage_rows(0, Kc[0], th4);
    stage_rows(QKPT, Qc[0], th4);
    fetch_rows(0, kg, 1, th4);
    fetch_rows(QKPT, qg, 1, th4);
    stage_rows(0, Kc[1], th4);
    stage_rows(QKPT, Qc[1], th4);
    fetch_rows(0, kg, 2, th4);
    fetch_rows(QKPT, qg, 2, th4);
  } else {  // T/V of chunk 0 staged, chunk 1 in flight; gates of chunks 0, 1 staged, chunk 2 in flight
    fetch_tv(0, th2);
    stage_tv(0, th2);
    fetch_tv(1, th2);
    if (w == 2) {
      fetch_gates(0);
      stage_gates(0);
      fetch_gates(1);
      stage_gates(1);
      fetch_gates(2);
    }
  }
  __syncthreads();
  if (nc > 0) {
    if (w < 2) {
      bf16x8 qf[KS][4];
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) qf[s2][tb] = ld8(Qc[0] + (16 * tb + li) * KP + 32 * s2 + 8 * g4);
      load_kf(0);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) Zt[tb] = f32x4{};
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) Zt[tb] = mma(sb(s2), qf[s2][tb], Zt[tb]);
    } else {
      run_p_side(0, lane);
    }
  }
  __syncthreads();

  // ------------------------------------------------------------------ chunk loop
  // Slots in use during step i: state waves read K_i, T_i, V_i, P_i, gates_i and Q_{i+1}, write
  // O_i; helpers read K_{i+1}, Q_{i+1}, gates_{i+1} (P_{i+1}) and O_{i-1}, write K_{i+2}, Q_{i+2},
  // T_{i+1}, V_{i+1}, P_{i+1}, gates_{i+2}. No slot is written and read in the same step.
  for (int i = 0; i < nc; ++i) {
    if (w < 2) {
      const bf16* kb = Kc[i % 3];
      const bf16* tp = Tb[i & 1];
      const bf16* vp = Vc[i & 1];
      const bf16* pp = Pb[i & 1];
      bf16* op = Ob[i & 1];
      const ChunkGates& G = gv[i % 3];

      // ---- 1: K reads for the second half of Y and the reads for X (V, beta, beta e^gam); Y = K S
      //      starts on the fragments read ahead in the previous step
      bf16x8 kf2[KS - KSH][4];
#pragma unroll
      for (int s2 = KSH; s2 < KS; ++s2)
#pragma unroll
        for (int b = 0; b < 4; ++b) kf2[s2 - KSH][b] = ld8(kb + (16 * b + li) * KP + 32 * s2 + 8 * g4);
      bf16x4 vv[4];
      float4 bt[4], bg[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        vv[b] = ld4_tr(vp, kVP, 16 * b, 16 * sw, lane);
        bt[b] = ld4f(&G.bet[16 * b + 4 * g4]);
        bg[b] = ld4f(&G.begam[16 * b + 4 * g4]);
      }
      phase();
      f32x4 D[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) D[b] = f32x4{};
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          D[b] = mma(s2 < KSH ? __builtin_bit_cast(bf16x8, KF[4 * s2 + b]) : kf2[s2 - KSH][b], sb(s2), D[b]);
      phase();
      // ---- 2: reads of T - I; X = beta V - beta e^gam Y (kept in fp32 as the Delta accumulator's start)
      bf16x8 tf[6];
      tf[0] = ld8(tp + li * kCP + 8 * g4);
      tf[1] = ld8(tp + (16 + li) * kCP + 8 * g4);
      tf[2] = ld8(tp + (32 + li) * kCP + 8 * g4);
      tf[3] = ld8(tp + (48 + li) * kCP + 8 * g4);
      tf[4] = ld8(tp + (32 + li) * kCP + 32 + 8 * g4);
      tf[5] = ld8(tp + (48 + li) * kCP + 32 + 8 * g4);
      phase();
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        D[b][0] = bt[b].x * (float)vv[b][0] - bg[b].x * D[b][0];
        D[b][1] = bt[b].y * (float)vv[b][1] - bg[b].y * D[b][1];
        D[b][2] = bt[b].z * (float)vv[b][2] - bg[b].z * D[b][2];
        D[b][3] = bt[b].w * (float)vv[b][3] - bg[b].w * D[b][3];
      }
      const bf16x8 xb0 = pack8(D[0], D[1]), xb1 = pack8(D[2], D[3]);
      phase();
      // ---- 3: reads of P, e^{gam_c - gam}, scale e^gam; Delta = X + (T - I) X (T - I vanishes above the diagonal)
      bf16x8 pf[6];
      float4 dla[2], dlb[2];
      float eg[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) pf[tb] = ld8(pp + (16 * tb + li) * kCP + 8 * g4);
      pf[4] = ld8(pp + (32 + li) * kCP + 32 + 8 * g4);
      pf[5] = ld8(pp + (48 + li) * kCP + 32 + 8 * g4);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        dla[u] = ld4f(&G.dlast[32 * u + 4 * g4]);
        dlb[u] = ld4f(&G.dlast[32 * u + 16 + 4 * g4]);
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) eg[tb] = G.egam[16 * tb + li];
      const float ec = __expf(G.gam[kC - 1]);
      phase();
      D[0] = mma(tf[0], xb0, D[0]);
      D[1] = mma(tf[1], xb0, D[1]);
      D[2] = mma(tf[2], xb0, D[2]);
      D[3] = mma(tf[3], xb0, D[3]);
      D[2] = mma(tf[4], xb1, D[2]);
      D[3] = mma(tf[5], xb1, D[3]);
      const bf16x8 db0 = pack8(D[0], D[1]), db1 = pack8(D[2], D[3]);
      phase();
      // ---- 4: K^T reads for the first half of the state tiles; O^T = scale e^gam Z^T + Delta^T
      //      (scale P)^T -> Ob[token][column]; Delta~ = e^{gam_c - gam} Delta as bf16 hi + lo
      constexpr int KH = KT / 2;
      bf16x8 ktf[KT][2];
#pragma unroll
      for (int a = 0; a < KH; ++a)
#pragma unroll
        for (int u = 0; u < 2; ++u) ktf[a][u] = ld8_tr_pair(kb, KP, 32 * u, 32 * (a >> 1) + 4 * (a & 1), lane);
      phase();
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 o = Zt[tb] * (p.scale * eg[tb]);
        o = mma(db0, pf[tb], o);
        if (tb >= 2) o = mma(db1, pf[tb + 2], o);
        *reinterpret_cast<bf16x4*>(op + (16 * tb + li) * kVP + 16 * sw + 4 * g4) = to_bf16x4(o[0], o[1], o[2], o[3]);
      }
      bf16x8 dh[2], dl[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f32x4 x0 = {dla[u].x * D[2 * u][0], dla[u].y * D[2 * u][1], dla[u].z * D[2 * u][2], dla[u].w * D[2 * u][3]};
        const f32x4 x1 = {dlb[u].x * D[2 * u + 1][0], dlb[u].y * D[2 * u + 1][1], dlb[u].z * D[2 * u + 1][2],
                          dlb[u].w * D[2 * u + 1][3]};
        split8(x0, x1, dh[u], dl[u]);
      }
      phase();
      // ---- 5: K^T reads for the second half; S' = e^{gam_c} S + K^T Delta~ on the first half
#pragma unroll
      for (int a = KH; a < KT; ++a)
#pragma unroll
        for (int u = 0; u < 2; ++u) ktf[a][u] = ld8_tr_pair(kb, KP, 32 * u, 32 * (a >> 1) + 4 * (a & 1), lane);
      phase();
#pragma unroll
      for (int a = 0; a < KH; ++a) {
        S[a] *= ec;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          S[a] = mma(ktf[a][u], dh[u], S[a]);
          S[a] = mma(ktf[a][u], dl[u], S[a]);
        }
      }
      phase();
      // ---- 6: Q reads of the next chunk (first half of the key steps); the second half of the
      //      update; S in bf16
      const bool more = i + 1 < nc;
      const bf16* qb = Qc[(i + 1) & 1];
      bf16x8 qf[KS][4];
      if (more) {
#pragma unroll
        for (int s2 = 0; s2 < KSH; ++s2)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) qf[s2][tb] = ld8(qb + (16 * tb + li) * KP + 32 * s2 + 8 * g4);
      }
      phase();
#pragma unroll
      for (int a = KH; a < KT; ++a) {
        S[a] *= ec;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          S[a] = mma(ktf[a][u], dh[u], S[a]);
          S[a] = mma(ktf[a][u], dl[u], S[a]);
        }
      }
      make_sb();
      phase();
      // ---- 7: the other Q reads and the K reads for the next Y; Z^T = S^T Q^T of the next chunk
      if (more) {
#pragma unroll
        for (int s2 = KSH; s2 < KS; ++s2)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) qf[s2][tb] = ld8(qb + (16 * tb + li) * KP + 32 * s2 + 8 * g4);
        load_kf(i + 1);
        phase();
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) Zt[tb] = f32x4{};
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) Zt[tb] = mma(sb(s2), qf[s2][tb], Zt[tb]);
      }
    } else if (w >= 4) {
      const int tq = opaque_int(th4);
      if (i > 0) store_o(i - 1, tq);
      stage_rows(0, Kc[(i + 2) % 3], tq);
      stage_rows(QKPT, Qc[i & 1], tq);
      fetch_rows(0, kg, i + 3, tq);
      fetch_rows(QKPT, qg, i + 3, tq);
      if (i + 1 < nc) run_p_side(i + 1, opaque_int(lane));
    } else {
      const int tq = opaque_int(th2);
      stage_tv((i + 1) & 1, tq);
      if (w == 2) stage_gates(i + 2);
      fetch_tv(i + 2, tq);
      if (w == 2) fetch_gates(i + 3);
      if (i + 1 < nc) run_p_side(i + 1, opaque_int(lane));
    }
    __syncthreads();
  }
  if (w >= 4 && nc > 0) store_o(nc - 1, th4);

  if (p.ht && w < 2) {
#pragma unroll
    for (int a = 0; a < KT; ++a) {
      const int kd0 = 32 * (a >> 1) + 8 * g4 + 4 * (a & 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) p.ht[sbase + (int64_t)(kd0 + r) * VD + li] = S[a][r];
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
